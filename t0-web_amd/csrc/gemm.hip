// Quantized-weight GEMM for gfx950 (CDNA4): llama.cpp Q8_0/Q4_0 blocks (and
// f16 rows) are read verbatim from HBM and dequantized inside the kernel.
//
// Two kernels implement the t0-fast `linear()` contract (crates/t0-fast/src/
// model.rs:406-504; ops.rs:40-42, y = x W^T + b):
//
//  * k_gemm — MFMA tile kernel for large M: 128x128, 256x128 or 256x256 output
//    tiles per 4-wave workgroup, v_mfma_f32_32x32x16_f16.  Per 64-wide K step
//    each thread fetches 32-value weight blocks (34 B Q8_0 / 18 B Q4_0 / 64 B
//    f16) and 32-value activation strips into registers two steps ahead, then
//    dequantizes the blocks to f16 with packed f16 math (exact integer-to-f16
//    via the 0x6400 exponent trick, then one rounding of d*q) into a
//    double-buffered LDS tile.  Accumulation is f32.
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
#include <type_traits>

#include "kernels.h"
#include "lanes.h"
#include "t0hip_internal.h"

namespace t0h {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// Four dwords at a 4-byte-aligned address (a Q8_0 / Q4_0 span): still one 16-byte load on gfx950,
// without the 16-byte alignment a uint4 access would promise the compiler.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int TK = 64, LDK = TK + 8;

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
// MFMA tile kernel.  Four waves (2 x 2); each wave owns TI x TJ tiles of
// v_mfma_f32_32x32x16_f16, so the workgroup tile is (64*TI) x (64*TJ) x 64.
// Larger wave tiles cut LDS bytes per flop (the main loop's limiter): 128x128
// waves (TI = TJ = 4) read half the LDS bytes per MFMA of 64x64 waves, and
// keep their 256 accumulators in AGPRs at one wave per SIMD.
// Measured on MI355X: 32x32x16 sustains ~2.2 PFLOP/s even at one wave per SIMD,
// where 16x16x32 needs 16+ independent chains and several waves.
// ---------------------------------------------------------------------------
template <int TI, int TJ>
struct Tile {
  static constexpr int BM = 64 * TI, BN = 64 * TJ;    // workgroup tile
  static constexpr int RA = BM / 128, RB = BN / 128;  // A / weight rows per loader thread
  static constexpr int WPE = TI * TJ > 4 ? 1 : 2;     // waves per SIMD the registers allow
  static constexpr int LDS_MAIN = 2 * (BM + BN) * LDK * 2;
  static constexpr int LDS_EPI = 4 * 32 * (TJ * 32 + 4) * 4;
  static constexpr int LDS = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
};

// Raw bytes of one thread's weight share of a K step: half of the step (one
// 32-value block, `part` 0 or 1) of one row.
template <int WT, bool AL4>
__device__ __forceinline__ void load_w(const uint8_t* wrow, int kt, int part, uint32_t (&br)[16]) {
  if (WT == T0H_F16) {
    const uint4* src = reinterpret_cast<const uint4*>(wrow + (size_t)(kt * TK + part * 32) * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 v = src[i];
      br[4 * i + 0] = v.x;
      br[4 * i + 1] = v.y;
      br[4 * i + 2] = v.z;
      br[4 * i + 3] = v.w;
    }
    return;
  }
  constexpr int BB = block_bytes(WT);
  if (AL4) {  // the step's two blocks start 4-byte aligned: dword loads, realigned in dequant_w
    const uint32_t* src = reinterpret_cast<const uint32_t*>(wrow) + (WT == T0H_Q8_0 ? 17 * kt + 8 * part : 9 * kt + 4 * part);
    constexpr int NW = WT == T0H_Q8_0 ? 9 : 5;
#pragma unroll
    for (int i = 0; i < NW; ++i) br[i] = src[i];
  } else {
    const uint16_t* src = reinterpret_cast<const uint16_t*>(wrow + (size_t)(2 * kt + part) * BB);
    constexpr int NQ = WT == T0H_Q8_0 ? 8 : 4;
    br[0] = src[0];
#pragma unroll
    for (int i = 0; i < NQ; ++i) br[1 + i] = (uint32_t)src[1 + 2 * i] | ((uint32_t)src[2 + 2 * i] << 16);
  }
}

// One block (32 values, k order) to packed f16 in out[0..15].
template <int WT, bool AL4>
__device__ __forceinline__ void dequant_w(const uint32_t (&br)[16], int part, uint32_t (&out)[16]) {
  if (WT == T0H_F16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = br[i];
    return;
  }
  uint32_t dbits, q[8];
  constexpr int NQ = WT == T0H_Q8_0 ? 8 : 4;
  if (AL4) {
    // part 0: the block starts at byte 0 of br (scale in the low half of br[0]);
    // part 1: at byte 2 (Q8_0 34 = 8*4+2, Q4_0 18 = 4*4+2), scale in the high half.
    const uint32_t sel = part ? 0x07060504u : 0x05040302u;
    dbits = part ? (br[0] >> 16) : (br[0] & 0xffffu);
#pragma unroll
    for (int i = 0; i < NQ; ++i) q[i] = perm(br[i + 1], br[i], sel);
  } else {
    dbits = br[0] & 0xffffu;
#pragma unroll
    for (int i = 0; i < NQ; ++i) q[i] = br[1 + i];
  }
  const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)dbits);
  const half2v dd = {dh, dh};
  if (WT == T0H_Q8_0) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) q8x4_f16(q[i], dd, out[2 * i], out[2 * i + 1]);
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      q4x4_f16(q[i] & 0x0f0f0f0fu, dd, out[2 * i], out[2 * i + 1]);                 // values 4i..4i+3
      q4x4_f16((q[i] >> 4) & 0x0f0f0f0fu, dd, out[8 + 2 * i], out[8 + 2 * i + 1]);  // values 16+4i..
    }
  }
}

// The same dequantization split into chunks (one quant dword each) so the
// VALU work can be spread between MFMAs.  Q8_0: 8 chunks of 4 values;
// Q4_0: 4 chunks of 8 values (4 low nibbles -> k 4c.., 4 high -> k 16+4c..).
template <int WT>
constexpr int dq_chunks() { return WT == T0H_Q8_0 ? 8 : (WT == T0H_Q4_0 ? 4 : 0); }

template <int WT, bool AL4>
__device__ __forceinline__ half2v dq_scale(const uint32_t (&br)[16], int part) {
  const uint32_t dbits = AL4 ? (part ? (br[0] >> 16) : (br[0] & 0xffffu)) : (br[0] & 0xffffu);
  const _Float16 dh = __builtin_bit_cast(_Float16, (uint16_t)dbits);
  return half2v{dh, dh};
}

template <int WT, bool AL4>
__device__ __forceinline__ void dq_chunk(const uint32_t (&br)[16], int part, int c, half2v dd, uint32_t (&out)[16]) {
  const uint32_t q = AL4 ? perm(br[c + 1], br[c], part ? 0x07060504u : 0x05040302u) : br[1 + c];
  if (WT == T0H_Q8_0) {
    q8x4_f16(q, dd, out[2 * c], out[2 * c + 1]);
    asm volatile("" : "+v"(out[2 * c]), "+v"(out[2 * c + 1]));  // keep the chunk here
  } else {
    q4x4_f16(q & 0x0f0f0f0fu, dd, out[2 * c], out[2 * c + 1]);
    q4x4_f16((q >> 4) & 0x0f0f0f0fu, dd, out[8 + 2 * c], out[8 + 2 * c + 1]);
    asm volatile("" : "+v"(out[2 * c]), "+v"(out[2 * c + 1]), "+v"(out[8 + 2 * c]), "+v"(out[8 + 2 * c + 1]));
  }
}

// Epilogue shared by the MFMA tile kernels, staged through LDS: each wave
// writes a 32-row slice of its results (bias, SwiGLU applied) as f32 into its
// own LDS region, then streams the slice out in 16-byte row chunks (coalesced
// f32/f16 stores, vector residual read-modify-write).  acc[i][j] is the wave's
// 32x32 tile (rows row_base + 32 i, tile column group j); in each tile lane l
// holds column l%32, rows (e/4)*8 + (l/32)*4 + e%4.  SwiGLU: groups j < TJ/2
// are gate columns and j + TJ/2 the up columns of the same hidden units, so the
// wave writes TJ*16 output columns from cbase; otherwise TJ*32.  `smemf` needs
// (waves) * 32 * (W + 4) floats and must be free (callers end their main loop
// with a barrier).
// Bias of the one column a lane writes when a wave has one column group (b1:
// the up half of SwiGLU; 0 past N or without bias), for kernels that load it
// before their main loop and hand it to store_tile (PRE) so that the epilogue
// does not start with a memory round trip.
template <int EPI>
__device__ __forceinline__ void tile_bias1(const GemmDesc& d, int lane, int cbase, float& b0, float& b1) {
  const int lc = lane & 31, col = cbase + (EPI == EPI_SWIGLU_F16 ? (lc & 15) : lc);
  const bool ok = d.bias && col < d.N;
  b0 = ok ? d.bias[col] : 0.0f;
  b1 = (EPI == EPI_SWIGLU_F16 && ok) ? d.bias[d.N + col] : 0.0f;
}

// RN (split RMSNorm, see GemmDesc): 0 none; 1 consumer: rs holds the scale of
// each of the tile's rows (rs[32 i + r] for row row_base + 32 i + r), applied to
// the accumulators before the bias; 2 producer (EPI_RESID_F32, vector stores,
// N % 32 == 0): the residual rows' f16 norm input and partial sums of squares.
// PREO (TI == 1, one 32-column group, vector stores): the caller loaded the
// residual's old rows (old_pre, as load_old below) and the producer's norm scales
// (g_pre, the four columns of each chunk) before its main loop.
template <int EPI, int TI, int TJ, bool PRE = false, int RN = 0, bool PREO = false>
__device__ __forceinline__ void store_tile(const GemmDesc& d, floatx16 (&acc)[TI][TJ], float* smemf, int wave,
                                           int lane, int row_base, int cbase, float pre0 = 0.0f,
                                           float pre1 = 0.0f, const float* rs = nullptr,
                                           const float4* old_pre = nullptr, const float4* g_pre = nullptr) {
  static_assert(!PREO || (TI == 1 && TJ == 1 && EPI == EPI_RESID_F32), "preloaded rows: one residual slice");
  static_assert(RN != 1 || EPI != EPI_RESID_F32, "a residual epilogue is not a norm consumer");
  static_assert(RN != 2 || EPI == EPI_RESID_F32, "only a residual epilogue produces the norm");
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  static_assert(!PRE || TJ == 1, "a preloaded bias covers one column group");
  // SwiGLU with one column group (PAIR): lanes l%32 < 16 hold the gate and
  // lanes l%32 >= 16 the up column of the same 16 hidden units.
  constexpr bool PAIR = SWI && TJ == 1;
  constexpr int W = PAIR ? 16 : (SWI ? TJ * 16 : TJ * 32);  // output columns per wave
  constexpr int SLD = W + 4;                                 // staging row stride (floats)
  constexpr int NJ = SWI && !PAIR ? TJ / 2 : TJ;             // staged column groups per wave
  const int M = d.M, N = d.N;
  float* stage = smemf + wave * 32 * SLD;
  const int lc = lane & 31, lr = (lane >> 5) * 4, uc = PAIR ? (lc & 15) : lc;
  // row scale of accumulator element e of slice i (1 without a split RMSNorm)
  auto rsc = [&](int i, int e) {
    if constexpr (RN == 1)
      return rs[i * 32 + (e >> 2) * 8 + lr + (e & 3)];
    else
      return 1.0f;
  };
  float b0[NJ], b1[NJ];
  if constexpr (PRE) {
    b0[0] = pre0;
    b1[0] = pre1;
  } else {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int col = cbase + j * 32 + uc;
      const bool ok = d.bias && col < N;
      b0[j] = ok ? d.bias[col] : 0.0f;
      b1[j] = (SWI && ok) ? d.bias[N + col] : 0.0f;
    }
  }
  const bool vec_ok = (d.ldy & 3) == 0 && (N & 3) == 0;
  // f16 outputs of one column group (the register-operand and medium-M
  // kernels) in 16-byte chunks: adjacent columns sit in lanes l and l^1 with the
  // same rows, so one DPP swap pairs them into f16 dwords; each slice is staged
  // as f16 (half the LDS traffic of the f32 stage) and stored 8 columns a lane.
  constexpr bool F16P = PAIR || (EPI == EPI_STORE_F16 && TJ == 1);
  if constexpr (F16P) {
    const bool vec8 = (d.ldy & 7) == 0 && (N & 7) == 0 && (reinterpret_cast<uintptr_t>(d.y) & 15) == 0;
    if (vec8) {
      constexpr int WD = W / 2, SH = WD + 4;  // f16 dwords per staged row (+4: 16-byte aligned rows)
      constexpr int CPR = WD / 4;             // 16-byte chunks per row
      static_assert(SH <= SLD, "f16 stage fits the f32 stage");
      uint32_t* st = reinterpret_cast<uint32_t*>(stage);
      const int odd = lc & 1;
      auto pack = [&](float mine, float nb) {
        const half2v pr = odd ? half2v{(_Float16)nb, (_Float16)mine} : half2v{(_Float16)mine, (_Float16)nb};
        return __builtin_bit_cast(uint32_t, pr);
      };
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        if constexpr (PAIR) {
          // result k of lane l: unit l%16, row of e = 2k + (l%32)/16 (as below)
          float v[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const auto gu = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[i][0][2 * k]),
                                                             __float_as_uint(acc[i][0][2 * k + 1]), false, false);
            const float sc = rsc(i, 2 * k + (lc >> 4));
            v[k] = silu(__uint_as_float(gu[0]) * sc + b0[0]) * (__uint_as_float(gu[1]) * sc + b1[0]);
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const float nb = dpp_move<0xB1>(v[k]);  // lane l^1
            if ((k & 1) == odd) {
              const int ee = 2 * k + (lc >> 4);
              st[((ee >> 2) * 8 + lr + (ee & 3)) * SH + (uc >> 1)] = pack(v[k], nb);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            float v = acc[i][0][e] * rsc(i, e) + b0[0];
            if (d.relu) v = fmaxf(v, 0.0f);
            const float nb = dpp_move<0xB1>(v);  // lane l^1
            if ((e & 1) == odd) st[((e >> 2) * 8 + lr + (e & 3)) * SH + (lc >> 1)] = pack(v, nb);
          }
        }
        const int row0 = row_base + i * 32;
#pragma unroll
        for (int t = 0; t < 32 * CPR / 64; ++t) {
          const int idx = t * 64 + lane, r = idx / CPR, c = idx % CPR;
          const int row = row0 + r, col = cbase + c * 8;
          if (row < M && col < N)
            *reinterpret_cast<uint4*>(static_cast<_Float16*>(d.y) + (size_t)row * d.ldy + col) =
                *reinterpret_cast<const uint4*>(st + r * SH + c * 4);
        }
      }
      return;
    }
  }
  // Residual: the old values of a 32-row slice are loaded one slice ahead, so
  // the read-modify-writes do not wait on a memory round trip each.
  // (Wide waves, NT > 8, load each slice's own values before staging it.)
  constexpr int NT = W / 8;  // 16-byte chunks per lane per slice
  constexpr bool RES = EPI == EPI_RESID_F32, RES2 = RES && NT <= 8;
  float4 yo[RES2 ? 2 : 1][RES ? NT : 1];
  auto load_old = [&](int i, float4 (&dst)[RES ? NT : 1]) {
    if constexpr (RES) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const int idx = t * 64 + lane, row = row_base + i * 32 + idx / (W / 4), col = cbase + (idx % (W / 4)) * 4;
        dst[t] = row < M && col < N ? *reinterpret_cast<const float4*>(static_cast<const float*>(d.y) +
                                                                       (size_t)row * d.ldy + col)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  };
  if constexpr (PREO) {
#pragma unroll
    for (int t = 0; t < NT; ++t) yo[0][t] = old_pre[t];
  } else if (RES2 && vec_ok) {
    load_old(0, yo[0]);
  }
  // Each wave stages into and reads back from its own region, and a wave's
  // LDS operations complete in order: no barrier is needed.
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    if (RES2 && vec_ok && i + 1 < TI) load_old(i + 1, yo[(i + 1) & 1]);
    if (RES && !RES2 && vec_ok) load_old(i, yo[0]);
    if constexpr (PAIR) {
      // Results e and e+1 swap across the 16-lane rows: rows 0/2 (gate lanes)
      // end with (gate, up) of result e, rows 1/3 (up lanes) with those of
      // result e+1, so every lane forms one distinct output of unit l%16.
#pragma unroll
      for (int e = 0; e < 16; e += 2) {
        const auto gu = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc[i][0][e]),
                                                         __float_as_uint(acc[i][0][e + 1]), false, false);
        const int ee = e + (lc >> 4);
        const float sc = rsc(i, ee);
        const float v = silu(__uint_as_float(gu[0]) * sc + b0[0]) * (__uint_as_float(gu[1]) * sc + b1[0]);
        stage[((ee >> 2) * 8 + lr + (ee & 3)) * SLD + uc] = v;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int r = (e >> 2) * 8 + lr + (e & 3);
        const float sc = rsc(i, e);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
          stage[r * SLD + j * 32 + lc] = SWI ? silu(acc[i][j][e] * sc + b0[j]) * (acc[i][j + TJ / 2][e] * sc + b1[j])
                                             : acc[i][j][e] * sc + b0[j];
      }
    }
    const int row0 = row_base + i * 32;
#pragma unroll
    for (int t = 0; t < W / 8; ++t) {
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
        if ((EPI == EPI_STORE_F32 || EPI == EPI_STORE_F16) && d.relu) {
          v.x = fmaxf(v.x, 0.0f); v.y = fmaxf(v.y, 0.0f); v.z = fmaxf(v.z, 0.0f); v.w = fmaxf(v.w, 0.0f);
        }
        if constexpr (RES) {
          const float4 old = yo[RES2 ? (i & 1) : 0][t];
          const float4 nx = make_float4(old.x + v.x, old.y + v.y, old.z + v.z, old.w + v.w);
          *reinterpret_cast<float4*>(static_cast<float*>(d.y) + o) = nx;
          if constexpr (RN == 2) {  // split RMSNorm producer (N % 32 == 0: a 32-column group's 8 lanes are all here)
            const float4 g4 = PREO ? g_pre[t] : *reinterpret_cast<const float4*>(d.norm_g + col);
            const half4 hn = {(_Float16)(nx.x * g4.x * RN_SCALE), (_Float16)(nx.y * g4.y * RN_SCALE),
                              (_Float16)(nx.z * g4.z * RN_SCALE), (_Float16)(nx.w * g4.w * RN_SCALE)};
            *reinterpret_cast<half4*>(d.norm_out + (size_t)row * N + col) = hn;
            const float sq = lane_sum8((nx.x * nx.x + nx.y * nx.y) + (nx.z * nx.z + nx.w * nx.w));
            if ((lane & 7) == 0) d.norm_ssq[(size_t)row * (N / 32) + col / 32] = sq;
          }
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
          if ((EPI == EPI_STORE_F32 || EPI == EPI_STORE_F16) && d.relu) x = fmaxf(x, 0.0f);
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
  }
}

template <int WT, bool A32, int EPI, bool K64, int TI, int TJ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(Tile<TI, TJ>::WPE, Tile<TI, TJ>::WPE)))
void k_gemm(const GemmDesc d) {
  using C = Tile<TI, TJ>;
  constexpr int BM = C::BM, BN = C::BN, RA = C::RA, RB = C::RB;
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  constexpr int HB = SWI ? BN / 2 : BN;  // output columns per tile (SwiGLU: gate rows then up rows)
  extern __shared__ __align__(16) _Float16 smem[];
  _Float16* As = smem;                 // [2][BM][LDK]
  _Float16* Bs = smem + 2 * BM * LDK;  // [2][BN][LDK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = d.M, N = d.N, K = d.K;
  const int tiles_n = (N + HB - 1) / HB;

  // XCD-aware remap: blocks are dispatched round-robin over 8 XCDs; give each
  // XCD a contiguous range of logical tiles (N fastest within an M strip), so
  // an activation strip is fetched once per XCD and shared through its L2.
  const int total = gridDim.x, bid = blockIdx.x;
  const int per = total / 8;
  const int logical = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
  const int tm = logical / tiles_n, tn = logical % tiles_n;
  const int m0 = tm * BM;

  // Loader roles: thread t moves rows t/2 + 128 r of both tiles, half t%2 of
  // each 64-wide K step (32 activations; one 32-value weight block).  Rows
  // past M read row M-1 and weight rows past N read row 0: their outputs are
  // never stored, and the loads stay branch-free.
  // f16 activations with K % 64 == 0 (ROWA) load by row instead: lanes
  // 8j..8j+7 of a wave read the 128 bytes of one row, so each 16-byte load
  // instruction covers 8 whole cache lines (the half-row split above touches
  // 32 lines per instruction, and the L1 tag lookups bound the main loop).
  // Thread t moves 16-byte chunk t%8 of rows t/8 + 32 q + 128 r.
  constexpr bool ROWA = !A32 && K64;
  const int lrow = tid >> 1, lh = tid & 1;
  const int arow = tid >> 3, achunk = tid & 7;
  const char* abase[RA][ROWA ? 4 : 1];
#pragma unroll
  for (int r = 0; r < RA; ++r) {
    if constexpr (ROWA) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        abase[r][q] = static_cast<const char*>(d.a) + (size_t)min(m0 + arow + 32 * q + 128 * r, M - 1) * d.lda * 2 +
                      achunk * 16;
    } else {
      abase[r][0] = static_cast<const char*>(d.a) + (size_t)min(m0 + lrow + 128 * r, M - 1) * d.lda * (A32 ? 4 : 2);
    }
  }
  const size_t rowb = WT == T0H_F16 ? (size_t)K * 2 : (size_t)(K / 32) * block_bytes(WT);
  const uint8_t* wbase[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int br = lrow + 128 * r;
    int wrow;
    bool ok;
    if (SWI) {
      const int g = tn * HB + (br % HB);
      ok = g < N;
      wrow = br < HB ? g : N + g;  // gate rows then up rows (the weight has 2N rows)
    } else {
      wrow = tn * BN + br;
      ok = wrow < N;
    }
    wbase[r] = static_cast<const uint8_t*>(d.w) + (size_t)(ok ? wrow : 0) * rowb;
  }

  // Raw global data of one K step, held in registers from its load to its LDS
  // store.  Two steps are in flight (loads for kt+2 issue while kt multiplies).
  struct Stage {
    uint32_t a[RA][A32 ? 32 : 16];
    uint32_t b[RB][16];
  };

  // K64 (K % 64 == 0, the model's shapes): no K tail, so loads and stores are
  // unconditional; otherwise the tail half of the last step reads the step's
  // first half again and is zeroed at the store.
  auto load_global = [&](Stage& st, int kt) {
    const int k0 = kt * TK + lh * 32;
    const int k0c = (K64 || k0 < K) ? k0 : k0 - 32;
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      if constexpr (ROWA) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint4 v = *reinterpret_cast<const uint4*>(abase[r][q] + kt * (TK * 2));
          st.a[r][4 * q + 0] = v.x;
          st.a[r][4 * q + 1] = v.y;
          st.a[r][4 * q + 2] = v.z;
          st.a[r][4 * q + 3] = v.w;
        }
      } else if (A32) {
        const float4* src = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(abase[r][0]) + k0c);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float4 v = src[i];
          st.a[r][4 * i + 0] = __builtin_bit_cast(uint32_t, v.x);
          st.a[r][4 * i + 1] = __builtin_bit_cast(uint32_t, v.y);
          st.a[r][4 * i + 2] = __builtin_bit_cast(uint32_t, v.z);
          st.a[r][4 * i + 3] = __builtin_bit_cast(uint32_t, v.w);
        }
      } else {
        const uint4* src = reinterpret_cast<const uint4*>(reinterpret_cast<const _Float16*>(abase[r][0]) + k0c);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint4 v = src[i];
          st.a[r][4 * i + 0] = v.x;
          st.a[r][4 * i + 1] = v.y;
          st.a[r][4 * i + 2] = v.z;
          st.a[r][4 * i + 3] = v.w;
        }
      }
    }
    const int part = (K64 || k0 < K) ? lh : 0;
#pragma unroll
    for (int r = 0; r < RB; ++r) load_w<WT, K64>(wbase[r], kt, part, st.b[r]);
  };

  // A stage's registers -> f16 tile rows (A converted or copied, weights
  // dequantized; the K tail zeroed), then into LDS buffer `buf`.
  auto prep = [&](Stage& st, int kt, uint32_t (&ao)[RA][16], uint32_t (&wo)[RB][16]) {
    const bool ok = K64 || kt * TK + lh * 32 < K;
    const bool tail = !K64 && kt * TK + TK > K;  // uniform
#pragma unroll
    for (int r = 0; r < RA; ++r) {
      if (A32) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          half2v h = {(_Float16)__builtin_bit_cast(float, st.a[r][2 * i]),
                      (_Float16)__builtin_bit_cast(float, st.a[r][2 * i + 1])};
          ao[r][i] = __builtin_bit_cast(uint32_t, h);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) ao[r][i] = st.a[r][i];
      }
      if (tail) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ao[r][i] = ok ? ao[r][i] : 0u;
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      dequant_w<WT, K64>(st.b[r], ok ? lh : 0, wo[r]);
      if (tail) {
#pragma unroll
        for (int i = 0; i < 16; ++i) wo[r][i] = ok ? wo[r][i] : 0u;
      }
    }
  };
  // LDS offset (elements) of this thread's 16-byte A chunk q of row group r
  auto a_lds = [&](int r, int q) {
    return ROWA ? (arow + 32 * q + 128 * r) * LDK + achunk * 8 : (lrow + 128 * r) * LDK + lh * 32 + 8 * q;
  };
  auto write = [&](const uint32_t (&ao)[RA][16], const uint32_t (&wo)[RB][16], int buf) {
#pragma unroll
    for (int r = 0; r < RA; ++r)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint4*>(As + (size_t)buf * BM * LDK + a_lds(r, i)) =
            make_uint4(ao[r][4 * i], ao[r][4 * i + 1], ao[r][4 * i + 2], ao[r][4 * i + 3]);
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      uint4* dst = reinterpret_cast<uint4*>(Bs + (size_t)buf * BN * LDK + (lrow + 128 * r) * LDK + lh * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i) dst[i] = make_uint4(wo[r][4 * i], wo[r][4 * i + 1], wo[r][4 * i + 2], wo[r][4 * i + 3]);
    }
  };
  auto store_lds = [&](Stage& st, int buf, int kt) {
    uint32_t ao[RA][16], wo[RB][16];
    prep(st, kt, ao, wo);
    write(ao, wo, buf);
  };

  // B-tile rows of the wave's TJ column tiles.  SwiGLU: tiles j < TJ/2 are gate
  // columns and tile j + TJ/2 the up columns of the same hidden units.
  int bcol[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
    bcol[j] = SWI ? (j < TJ / 2 ? wn * (HB / 2) + j * 32 : HB + wn * (HB / 2) + (j - TJ / 2) * 32) : wn * (BN / 2) + j * 32;

  floatx16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Operand lane layout: lane l holds row (A) / column (B) l%32 and k-slots
  // (l/32)*8 .. +8 of the 16-wide K slice.
  auto compute = [&](int buf, int kk_lo = 0, int kk_hi = TK / 16) {
    const _Float16* At = As + (size_t)buf * BM * LDK + (wm * (BM / 2) + (lane & 31)) * LDK + (lane >> 5) * 8;
    const _Float16* Bt = Bs + (size_t)buf * BN * LDK + (lane & 31) * LDK + (lane >> 5) * 8;
    // Fragments of slice kk+1 are read while slice kk multiplies; the
    // scheduling fence keeps at most two slices of fragments live.
    half8 af[2][TI], bf[2][TJ];
    auto frags = [&](int kk, half8 (&a)[TI], half8 (&b)[TJ]) {
#pragma unroll
      for (int i = 0; i < TI; ++i) a[i] = *reinterpret_cast<const half8*>(At + i * 32 * LDK + kk * 16);
#pragma unroll
      for (int j = 0; j < TJ; ++j) b[j] = *reinterpret_cast<const half8*>(Bt + bcol[j] * LDK + kk * 16);
    };
    frags(kk_lo, af[kk_lo & 1], bf[kk_lo & 1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = kk_lo; kk < kk_hi; ++kk) {
      if (kk + 1 < kk_hi) frags(kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk & 1][i], bf[kk & 1][j], acc[i][j], 0, 0, 0);
      // order within the slice: the next slice's LDS reads first, then the MFMAs
      if (kk + 1 < kk_hi) __builtin_amdgcn_sched_group_barrier(0x100, TI + TJ, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, TI * TJ, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One step of the two-stage pipeline in a single scheduling region: issue
  // the loads of step kl into `ld`; multiply LDS buffer `buf`; dequantize stage
  // `st` (step ks) with its VALU work interleaved between the MFMAs (the
  // matrix core runs them concurrently); write it to the other buffer.
  auto step2 = [&](int buf, Stage& ld, int kl, Stage& st) {
    if constexpr (C::WPE == 2 && !A32 && WT != T0H_F16 && K64) {
      constexpr int NS = TK / 16, NMS = TI * TJ, NM = NMS * NS;
      constexpr int NCH = dq_chunks<WT>() * RB;  // dequant chunks of this thread's weight rows
      constexpr int NW = 4 * (RA + RB);          // 16-byte LDS writes of the next step
      load_global(ld, kl);
      half2v dd[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) dd[r] = dq_scale<WT, true>(st.b[r], lh);
      uint32_t wo[RB][16];
      _Float16* An = As + (size_t)(buf ^ 1) * BM * LDK;
      _Float16* Bn = Bs + (size_t)(buf ^ 1) * BN * LDK + lrow * LDK + lh * 32;
      const _Float16* At = As + (size_t)buf * BM * LDK + (wm * (BM / 2) + (lane & 31)) * LDK + (lane >> 5) * 8;
      const _Float16* Bt = Bs + (size_t)buf * BN * LDK + (lane & 31) * LDK + (lane >> 5) * 8;
      half8 af[2][TI], bf[2][TJ];
      auto frags = [&](int kk, half8 (&a)[TI], half8 (&b)[TJ]) {
#pragma unroll
        for (int i = 0; i < TI; ++i) a[i] = *reinterpret_cast<const half8*>(At + i * 32 * LDK + kk * 16);
#pragma unroll
        for (int j = 0; j < TJ; ++j) b[j] = *reinterpret_cast<const half8*>(Bt + bcol[j] * LDK + kk * 16);
      };
      frags(0, af[0], bf[0]);
      __builtin_amdgcn_sched_barrier(0);
      // Program order is issue order (fenced after every MFMA): each slice
      // first reads the next slice's fragments; the dequant chunks of the next
      // step ride behind the MFMAs of the first NS-1 slices, its LDS writes
      // behind those of the last slice (all reads of this step are issued by
      // then, and the writes go to the other buffer).
#pragma unroll
      for (int kk = 0; kk < NS; ++kk) {
        if (kk + 1 < NS) frags(kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
        for (int i = 0; i < TI; ++i)
#pragma unroll
          for (int j = 0; j < TJ; ++j) {
            const int mi = i * TJ + j, m = kk * NMS + mi;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk & 1][i], bf[kk & 1][j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int c = 0; c < NCH; ++c)
              if (c * (NM - NMS) / NCH == m) dq_chunk<WT, true>(st.b[c / dq_chunks<WT>()], lh, c % dq_chunks<WT>(),
                                                                 dd[c / dq_chunks<WT>()], wo[c / dq_chunks<WT>()]);
            if (kk == NS - 1) {
#pragma unroll
              for (int w = 0; w < NW; ++w)
                if (w * NMS / NW == mi) {
                  if (w < 4 * RA) {
                    const int r = w / 4, q = w % 4;
                    *reinterpret_cast<uint4*>(An + a_lds(r, q)) =
                        make_uint4(st.a[r][4 * q], st.a[r][4 * q + 1], st.a[r][4 * q + 2], st.a[r][4 * q + 3]);
                  } else {
                    const int r = (w - 4 * RA) / 4, q = (w - 4 * RA) % 4;
                    *reinterpret_cast<uint4*>(Bn + 128 * r * LDK + 8 * q) =
                        make_uint4(wo[r][4 * q], wo[r][4 * q + 1], wo[r][4 * q + 2], wo[r][4 * q + 3]);
                  }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
          }
      }
    }
  };

  const int KT = (K + TK - 1) / TK;
  if constexpr (C::WPE == 2 && !A32 && WT != T0H_F16 && K64) {
    // Two register stages: steps alternate between (LDS buffer 0, stage s0) and
    // (buffer 1, stage s1); the body covers two steps so the stage registers
    // are indexed statically.
    // Past the last step the loads re-read step KT-1 and the stores fill the
    // idle buffer with it: every load and store is unconditional, so the
    // compiler's wait counts let step kt+2's loads stay in flight.
    Stage s0, s1;
    const int last = KT - 1;
    load_global(s0, 0);
    load_global(s1, min(1, last));
    store_lds(s0, 0, 0);
    __syncthreads();
    // Pairs of steps with one loop exit (an exit between the two steps makes
    // the compiler copy the accumulators every step); an odd last step runs
    // after the loop.
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
      step2(0, s0, min(kt + 2, last), s1);
      __syncthreads();
      step2(1, s1, min(kt + 3, last), s0);
      __syncthreads();
    }
    if (kt < KT) {
      step2(0, s0, last, s1);
      __syncthreads();
    }
  } else {
    // One register stage: large tiles, f32 activations, f16 weights or a K tail.
    Stage s0;
    const int last = KT - 1;
    load_global(s0, 0);
    store_lds(s0, 0, 0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
      load_global(s0, min(kt + 1, last));
      compute(kt & 1);
      store_lds(s0, (kt + 1) & 1, min(kt + 1, last));
      __syncthreads();
    }
  }

  // LDS is free after the main loop's last barrier: stage the epilogue in it.
  store_tile<EPI, TI, TJ>(d, acc, reinterpret_cast<float*>(smem), wave, lane, m0 + wm * (BM / 2),
                          SWI ? tn * HB + wn * (HB / 2) : tn * BN + wn * (BN / 2));
}

// ---------------------------------------------------------------------------
// DMA tile kernel: 256x256x64 tiles for K % 64 == 0, f16 activations and
// Q8_0/Q4_0 weights (the model's layer shapes).  Four waves, each 128x128 as
// 4x4 tiles of v_mfma_f32_32x32x16_f16 with the 256 accumulators in AGPRs.
//  * Activation tiles go global -> LDS with global_load_lds_dwordx4 (no
//    registers, tracked by vmcnt), three buffers deep: step kt+2 is in flight
//    while kt multiplies.
//  * Weight blocks go global -> registers one step ahead, are dequantized in
//    chunks between the MFMAs of the current step and written as f16 to the
//    other of two weight buffers.
//  * LDS rows are 128 bytes, unpadded, with 16-byte chunk c of row r stored in
//    slot c ^ ((r >> 1) & 7): the DMA writes (8 rows per wave instruction), the
//    weight writes and the 32x32 operand reads are all free of bank conflicts.
// ---------------------------------------------------------------------------
constexpr int DM_BM = 256, DM_BN = 256, DM_ROWB = 128;  // tile rows / cols, LDS row bytes
constexpr int DM_ABUF = DM_BM * DM_ROWB, DM_BBUF = DM_BN * DM_ROWB;
constexpr int DM_LDS = 3 * DM_ABUF + 2 * DM_BBUF;  // 160 KiB

__device__ __forceinline__ int dm_slot(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

template <int WT, int EPI>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm_dma(const GemmDesc d) {
  constexpr int TI = 4, TJ = 4, RB = 2;
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  constexpr int HB = SWI ? DM_BN / 2 : DM_BN;
  extern __shared__ __align__(16) _Float16 smem[];
  char* const lds = reinterpret_cast<char*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int M = d.M, N = d.N, K = d.K;
  const int tiles_n = (N + HB - 1) / HB;
  const int total = gridDim.x, bid = blockIdx.x;
  const int per = total / 8;
  const int logical = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
  const int tm = logical / tiles_n, tn = logical % tiles_n;
  const int m0 = tm * DM_BM;
  const int KT = K / TK, last = KT - 1;

  // Activation DMA: wave w fills rows w*64 .. w*64+63 with 8 instructions of
  // 8 rows each; lane L writes slot L%8 of row +L/8, so it fetches chunk
  // (L%8) ^ swizzle(row).  Rows past M read row M-1.
  const char* asrc[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int row = wave * 64 + q * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ ((row >> 1) & 7);
    asrc[q] = static_cast<const char*>(d.a) + (size_t)min(m0 + row, M - 1) * d.lda * 2 + chunk * 16;
  }
  auto dma_a = [&](int kt, int buf) {
    char* dst = lds + buf * DM_ABUF + wave * 64 * DM_ROWB;
#pragma unroll
    for (int q = 0; q < 8; ++q)
      __builtin_amdgcn_global_load_lds(asrc[q] + kt * (TK * 2), dst + q * 8 * DM_ROWB, 16, 0, 0);
  };

  // Weight rows: thread t moves tile rows t/2 and t/2+128, block t%2 of each step.
  const int lrow = tid >> 1, lh = tid & 1;
  const size_t rowb = (size_t)(K / 32) * block_bytes(WT);
  const uint8_t* wbase[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int br = lrow + 128 * r;
    int wrow;
    bool ok;
    if (SWI) {
      const int g = tn * HB + (br % HB);
      ok = g < N;
      wrow = br < HB ? g : N + g;
    } else {
      wrow = tn * DM_BN + br;
      ok = wrow < N;
    }
    wbase[r] = static_cast<const uint8_t*>(d.w) + (size_t)(ok ? wrow : 0) * rowb;
  }
  struct WStage {
    uint32_t b[RB][16];
  };
  auto load_b = [&](WStage& st, int kt) {
#pragma unroll
    for (int r = 0; r < RB; ++r) load_w<WT, true>(wbase[r], kt, lh, st.b[r]);
  };
  auto write_b_chunk = [&](const uint32_t (&wo)[16], int r, int q, int buf) {
    const int br = lrow + 128 * r;
    *reinterpret_cast<uint4*>(lds + 3 * DM_ABUF + buf * DM_BBUF + br * DM_ROWB + dm_slot(br, lh * 4 + q) * 16) =
        make_uint4(wo[4 * q], wo[4 * q + 1], wo[4 * q + 2], wo[4 * q + 3]);
  };

  int bcol[TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
    bcol[j] = SWI ? (j < TJ / 2 ? wn * (HB / 2) + j * 32 : HB + wn * (HB / 2) + (j - TJ / 2) * 32) : wn * (DM_BN / 2) + j * 32;

  floatx16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

  // Operand reads: lane l takes row l%32 of each 32-row tile and 16-byte chunk
  // 2*kk + l/32; every tile row base is a multiple of 32, so the swizzle of the
  // lane's row is ((l%32) >> 1) & 7 throughout.
  const int swz = ((lane & 31) >> 1) & 7;
  int koff[TK / 16];
#pragma unroll
  for (int kk = 0; kk < TK / 16; ++kk) koff[kk] = (((2 * kk + (lane >> 5)) ^ swz) * 16);
  const int arow = (wm * (DM_BM / 2) + (lane & 31)) * DM_ROWB, brow = (lane & 31) * DM_ROWB;

  // Prologue: A(0), B(0) and A(1), B(1) in flight; B(0) dequantized into buffer 0.
  WStage w0, w1;
  dma_a(0, 0);
  load_b(w0, 0);
  dma_a(min(1, last), 1);
  load_b(w1, min(1, last));
  {
    uint32_t wo[RB][16];
#pragma unroll
    for (int r = 0; r < RB; ++r) dequant_w<WT, true>(w0.b[r], lh, wo[r]);
#pragma unroll
    for (int r = 0; r < RB; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) write_b_chunk(wo[r], r, q, 0);
  }
  // A(0) landed: its DMA precedes B(1)'s loads, which dequant_w above did not
  // wait for; wait for everything but the step-1 loads.
  __builtin_amdgcn_s_waitcnt((8 + RB * (WT == T0H_Q8_0 ? 3 : 2)) | (7 << 4) | (15 << 8));
  __syncthreads();

  // One step: DMA A(kt+2), load B(kt+2); multiply buffers (kt%3, kt&1);
  // dequantize B(kt+1) between the MFMAs and write it to buffer (kt+1)&1.
  auto step = [&](int kt, int abuf, WStage& cur, WStage& nxt) {
    constexpr int NS = TK / 16, NMS = TI * TJ, NM = NMS * NS;
    constexpr int NCHR = dq_chunks<WT>(), NCH = NCHR * RB;
    dma_a(min(kt + 2, last), (abuf + 2) % 3);
    load_b(nxt, min(kt + 2, last));
    half2v dd[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) dd[r] = dq_scale<WT, true>(cur.b[r], lh);
    uint32_t wo[RB][16];
    const char* At = lds + abuf * DM_ABUF + arow;
    const char* Bt = lds + 3 * DM_ABUF + (kt & 1) * DM_BBUF + brow;
    half8 af[2][TI], bf[2][TJ];
    auto frags = [&](int kk, half8 (&a)[TI], half8 (&b)[TJ]) {
#pragma unroll
      for (int i = 0; i < TI; ++i) a[i] = *reinterpret_cast<const half8*>(At + i * 32 * DM_ROWB + koff[kk]);
#pragma unroll
      for (int j = 0; j < TJ; ++j) b[j] = *reinterpret_cast<const half8*>(Bt + bcol[j] * DM_ROWB + koff[kk]);
    };
    frags(0, af[0], bf[0]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < NS; ++kk) {
      if (kk + 1 < NS) frags(kk + 1, af[(kk + 1) & 1], bf[(kk + 1) & 1]);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const int mi = i * TJ + j, m = kk * NMS + mi;
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk & 1][i], bf[kk & 1][j], acc[i][j], 0, 0, 0);
#pragma unroll
          for (int c = 0; c < NCH; ++c)
            if (c * (NM - NMS) / NCH == m) dq_chunk<WT, true>(cur.b[c / NCHR], lh, c % NCHR, dd[c / NCHR], wo[c / NCHR]);
          if (kk == NS - 1) {
#pragma unroll
            for (int w = 0; w < 4 * RB; ++w)
              if (w * NMS / (4 * RB) == mi) write_b_chunk(wo[w / 4], w / 4, w % 4, (kt + 1) & 1);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    // A(kt+1) landed (issued before B(kt+1), whose data the dequant consumed).
    __builtin_amdgcn_s_waitcnt((8 + RB * (WT == T0H_Q8_0 ? 3 : 2)) | (7 << 4) | (15 << 8));
    __syncthreads();
  };

  // KT is even (checked at launch): two steps per iteration, one loop exit.
  int abuf = 0;
  for (int kt = 0; kt < KT; kt += 2) {
    step(kt, abuf, w1, w0);
    abuf = abuf == 2 ? 0 : abuf + 1;
    step(kt + 1, abuf, w0, w1);
    abuf = abuf == 2 ? 0 : abuf + 1;
  }

  // The last steps re-issued DMA into idle buffers; all of it must land before
  // the epilogue reuses the LDS.
  __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8));
  __syncthreads();

  store_tile<EPI, TI, TJ>(d, acc, reinterpret_cast<float*>(smem), wave, lane, m0 + wm * (DM_BM / 2),
                          SWI ? tn * HB + wn * (HB / 2) : tn * DM_BN + wn * (DM_BN / 2));
}

// ---------------------------------------------------------------------------
// Register-operand tile kernel: 256x256x64 tiles for K % 64 == 0, f16
// activations and Q8_0/Q4_0 weights.  Eight waves side by side along N, each
// all 256 rows x 32 weight columns as 8 tiles of v_mfma_f32_32x32x16_f16
// (128 accumulators, two waves per SIMD, one workgroup per CU).
//  * Weights never pass through LDS: each lane loads the raw 18/34-byte block
//    of its own weight row and dequantizes it straight into the MFMA B
//    fragment, so every weight column is dequantized once per tile (about two
//    VALU instructions per MFMA).  Inside a 64-wide K step the k order is
//    permuted so that lane half h owns block h: MFMA slice c takes
//    k = 32h + 8c .. 32h + 8c + 7 of the step, i.e. the Q4_0 nibbles of qs
//    bytes 8(c%2) .. +7 (low for c < 2, high for c >= 2) or Q8_0 qs bytes
//    8c .. +7.  The activation fragments follow the same order, so every
//    product of the step is still summed once.  SwiGLU: lanes l%32 < 16 take
//    the gate rows and the others the up rows of the same 16 hidden units.
//  * Activations: row-coalesced 16-byte loads (8 lanes per 128-byte row) two
//    steps ahead into three LDS buffers.  Each A fragment feeds
//    one MFMA; fragments stream through a ring read RD MFMAs ahead, across
//    the step's barrier into the next step (whose buffer is complete).
//  * Between MFMAs: one ring read, a dequantization sub-step (about four VALU
//    instructions) after every other MFMA, and in the first slice the step's
//    global loads, one per MFMA.  Measured on MI355X, a wave's VALU work
//    beyond a few instructions per MFMA adds to the MFMA time instead of
//    overlapping it, and bursts of loads right after a barrier stall issue.
// ---------------------------------------------------------------------------
constexpr int BF_BM = 256;
// NWV waves of 32 weight columns each; 8 waves: three activation buffers
// (110,592 bytes, one workgroup per CU), 4 waves: two (73,728 bytes, two
// workgroups per CU, so one's epilogue overlaps the other's main loop).
template <int NWV, int BM = BF_BM>
struct BfCfg {
  static constexpr int BN = 32 * NWV, NBUF = NWV == 8 ? 3 : 2, ABUF = BM * LDK, LDS = NBUF * ABUF * 2;
};

// Split RMSNorm consumer: the scale of rows m0 .. m0 + n - 1 (rows past M use row
// M - 1) into dst, from each row's ssq_parts partial sums of squares summed in order.
// A row's partials (ssq_parts <= RN_MAX_PARTS, a multiple of 4, 16-byte aligned rows)
// are loaded with every 16-byte load issued before the first is summed.
constexpr int RN_MAX_PARTS = 32;
__device__ __forceinline__ void row_scales(const GemmDesc& d, int m0, int n, float* dst) {
  for (int t = threadIdx.x; t < n; t += blockDim.x) {
    const float4* p = reinterpret_cast<const float4*>(d.row_ssq + (size_t)min(m0 + t, d.M - 1) * d.ssq_parts);
    float4 v[RN_MAX_PARTS / 4];
#pragma unroll
    for (int q = 0; q < RN_MAX_PARTS / 4; ++q)
      if (4 * q < d.ssq_parts) v[q] = p[q];
    float ss = 0.0f;
#pragma unroll
    for (int q = 0; q < RN_MAX_PARTS / 4; ++q)
      if (4 * q < d.ssq_parts) ss = (((ss + v[q].x) + v[q].y) + v[q].z) + v[q].w;
    dst[t] = 1.0f / (RN_SCALE * sqrtf(ss / (float)d.ssq_dim + 1e-8f));
  }
}

typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));
// The dequantization sub-step (0..3) that follows MFMA i of a TI-MFMA slice, or -1.
__host__ __device__ constexpr int dq_sub_at(int i, int TI) {
  for (int q = 0; q < 4; ++q)
    if ((q * TI) / 4 == i) return q;
  return -1;
}
// An activation chunk as f16 for the LDS tile: f16 chunks as they are, f32
// chunks (8 values) rounded to f16.
__device__ __forceinline__ u32x4 a_f16(u32x4 r) { return r; }
__device__ __forceinline__ u32x4 a_f16(u32x8 r) {
  half8 h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (_Float16)__uint_as_float(r[e]);
  return __builtin_bit_cast(u32x4, h);
}

template <int WT, int EPI, int NWV, bool A32, int BM>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_bf(const GemmDesc d) {
  using C = BfCfg<NWV, BM>;
  constexpr int BN = C::BN, NBUF = C::NBUF, BF_ABUF = C::ABUF;
  constexpr int TI = BM / 32, TJ = 1;         // 32x32 tiles per wave
  constexpr int ACH = BM * 8 / (64 * NWV);    // 16-byte activation chunks per thread and step
  constexpr int AQS = BM / ACH;               // row stride between a thread's chunks
  constexpr int NMI = 4 * TI;                 // MFMAs per step
  constexpr int RING = 8, RD = 6;             // A fragment ring; RING divides NMI
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  constexpr int HB = SWI ? BN / 2 : BN;          // output columns per tile
  constexpr int NWD = WT == T0H_Q8_0 ? 9 : 5;    // raw dwords a lane needs per step
  constexpr int SWD = WT == T0H_Q8_0 ? 17 : 9;   // dwords of one row's two blocks (one step)
  static_assert(NMI % RING == 0 && RD < RING && ACH <= TI && TI >= 4, "step work placement");
  static_assert(NWV * 32 * ((SWI ? 16 : 32) + 4) * 4 <= C::LDS, "epilogue stage fits the LDS");
  extern __shared__ __align__(16) _Float16 smem[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, lc = lane & 31;
  const int M = d.M, N = d.N, K = d.K;
  const int tiles_n = (N + HB - 1) / HB;
  const int KT = K / TK, last = KT - 1;
  // XCD-aware remap (blocks are dispatched round-robin over 8 XCDs): each
  // XCD gets a contiguous range of logical tiles, N fastest, so concurrent
  // tiles share activation rows in that XCD's L2.
  const int total = gridDim.x, bid = blockIdx.x, per = total / 8;
  const int t = bid < per * 8 ? (bid % 8) * per + bid / 8 : bid;
  const int tn = t % tiles_n, m0 = (t / tiles_n) * BM;
  // Two workgroups share a CU here, and with equal tiles they would start, reach
  // their epilogues and store together for the whole launch.  The second one of
  // each CU in the first round (blocks 256 .. 511 on the 256 CUs) starts about
  // 7 us late, so that one's epilogue stores overlap the other's MFMAs (config-4
  // step 0.7-0.8 % shorter, A/B on two boxes; 3.4 or 10 us measured less).
  if constexpr (NWV == 4) {
    if (total > 512 && bid >= 256 && bid < 512) {
      __builtin_amdgcn_s_sleep(127);  // 127 x 64 cycles
      __builtin_amdgcn_s_sleep(127);
    }
  }

  // Activation chunk t%8 of rows t/8 + AQS q (rows past M read row M-1,
  // never stored) as byte offsets from the tile's first row; the lane's weight
  // row (rows past N read row 0) as a dword offset, plus the dwords
  // (h ? NWD-1 : 0) of each step's 2-block span.
  const int arow = tid >> 3, achunk = tid & 7;
  // f32 activations (A32): a chunk is the 32 bytes of the same 8 values, held raw
  // until its LDS store converts it to f16
  constexpr int AB = A32 ? 4 : 2;  // bytes per activation value
  using AR = std::conditional_t<A32, u32x8, u32x4>;
  const char* const a_tile = static_cast<const char*>(d.a) + (size_t)m0 * d.lda * AB;
  int aoff[ACH];
#pragma unroll
  for (int q = 0; q < ACH; ++q) aoff[q] = (min(m0 + arow + AQS * q, M - 1) - m0) * d.lda * AB + achunk * 8 * AB;
  int woff;
  {
    int wrow;
    bool ok;
    if (SWI) {
      const int g = tn * HB + wave * 16 + (lc & 15);
      ok = g < N;
      wrow = lc < 16 ? g : N + g;
    } else {
      wrow = tn * BN + wave * 32 + lc;
      ok = wrow < N;
    }
    woff = (ok ? wrow : 0) * ((K / 32) * block_bytes(WT) / 4) + h * (NWD - 1);
  }
  const uint32_t* const wbase = static_cast<const uint32_t*>(d.w);
  // block h starts 2 bytes into the lane's first dword (h = 0) or at its
  // second dword (h = 1), after the scale in the first dword's high half
  const uint32_t qsel = h ? 0x07060504u : 0x05040302u;
  const uint32_t dsel = h ? 0x03020302u : 0x01000100u;

  auto load_a = [&](AR& r, int kt, int q) { r = *reinterpret_cast<const AR*>(a_tile + kt * (TK * AB) + aoff[q]); };
  auto a_dst = [&](int buf, int q) {
    return reinterpret_cast<u32x4*>(smem + buf * BF_ABUF + (arow + AQS * q) * LDK + achunk * 8);
  };
  auto load_b = [&](uint32_t (&r)[NWD], int kt) {
    const uint32_t* src = wbase + (uint32_t)(woff + kt * SWD);  // NWD contiguous dwords
#pragma unroll
    for (int i = 0; i < NWD; ++i) r[i] = src[i];
  };
  const _Float16* afr_base = smem + lc * LDK + h * 32;
  auto read_a = [&](int buf, int c, int i) {
    return *reinterpret_cast<const half8*>(afr_base + buf * BF_ABUF + i * 32 * LDK + c * 8);
  };

  // B fragment of slice c from the lane's raw dwords r, in four sub-steps of
  // about four VALU instructions each.
  uint32_t ts[4];
  half2v tdd;
  auto dq = [&](const uint32_t (&r)[NWD], int c, int sub, half8& out) {
    if (sub == 0) {
      const int i = WT == T0H_Q8_0 ? 2 * c : 2 * (c & 1);
      uint32_t qa = perm(r[i + 1], r[i], qsel), qb = perm(r[i + 2], r[i + 1], qsel);
      if (WT == T0H_Q4_0) {
        if (c >= 2) {
          qa >>= 4;
          qb >>= 4;
        }
        qa &= 0x0f0f0f0fu;
        qb &= 0x0f0f0f0fu;
      } else {
        qa ^= 0x80808080u;
        qb ^= 0x80808080u;
      }
      ts[0] = qa;
      ts[1] = qb;
      tdd = __builtin_bit_cast(half2v, perm(r[0], r[0], dsel));
    } else if (sub == 1) {
      ts[2] = perm(0x64646464u, ts[1], 0x04010400u);
      ts[3] = perm(0x64646464u, ts[1], 0x04030402u);
      ts[1] = perm(0x64646464u, ts[0], 0x04030402u);
      ts[0] = perm(0x64646464u, ts[0], 0x04010400u);
    } else if (sub == 2) {
      const _Float16 o = (_Float16)(WT == T0H_Q8_0 ? 1152.0f : 1032.0f);
      const half2v off = {o, o};
#pragma unroll
      for (int e = 0; e < 4; ++e) ts[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, ts[e]) - off);
    } else {
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, ts[e]) * tdd);
      out = __builtin_bit_cast(half8, make_uint4(o[0], o[1], o[2], o[3]));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) asm volatile("" : "+v"(ts[e]));
  };

  // The residual epilogues (wO, w2) load their bias before the main loop:
  // measured 2 us faster on wO; the f16 and SwiGLU epilogues measured ~1.5 us
  // slower with it and load theirs in store_tile.
  constexpr bool PREB = EPI == EPI_RESID_F32;
  const int cbase = SWI ? tn * HB + wave * 16 : tn * BN + wave * 32;

  float pb0 = 0.0f, pb1 = 0.0f;
  if constexpr (PREB) tile_bias1<EPI>(d, lane, cbase, pb0, pb1);

  floatx16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[i][0][e] = 0.0f;
  uint32_t wr0[NWD], wr1[NWD];
  half8 ring[RING], bf[2];
  AR ar[ACH];

  int abuf = 0;
  // One step: slice c, MFMA i (m = c*TI + i): the ring read of fragment
  // m + RD (with three buffers, in step kt+1 once past the step: its buffer
  // is complete; with two, the next step reads its first RD fragments after
  // the barrier), B sub-steps spread over the slice (every other MFMA at 256 rows), the activation chunk
  // loads of step kt+NBUF-1 and the W(kt+1) load early in the first slices
  // (W first when the ACH = 8 chunk loads would push it into the second
  // slice: its data is needed in the last), the activation stores in the
  // last slice.
  //
  // With two buffers (EARLY), a chunk's load for step kt+2 is issued right
  // after its store for step kt+1, so a load has a whole step and the barrier
  // to land instead of three slices (QKV 2.6, w2 3.5, SwiGLU 1.6 us faster at
  // config 4).  Q8_0 SwiGLU keeps the loads in the first slice: the longer
  // live range spills there.
  constexpr int WPOS = ACH < TI ? ACH : 0, A0 = ACH < TI ? 0 : 1;
  constexpr bool EARLY = NBUF == 2 && !(WT == T0H_Q8_0 && SWI);
  auto step = [&](int kt, uint32_t (&cur)[NWD], uint32_t (&nxt)[NWD]) {
    const int b1 = abuf + 1 == NBUF ? 0 : abuf + 1, b2 = b1 + 1 == NBUF ? 0 : b1 + 1;
    const int kb = min(kt + 1, last), ka = min(kt + NBUF - 1, last), ka2 = min(kt + 2, last);
    if constexpr (NBUF == 2) {
#pragma unroll
      for (int m = 0; m < RD; ++m) ring[m] = read_a(abuf, m / TI, m % TI);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int p = c & 1, n = p ^ 1;
#pragma unroll
      for (int i = 0; i < TI; ++i) {
        const int m = c * TI + i, mr = m + RD;
        acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ring[m % RING], bf[p], acc[i][0], 0, 0, 0);
        if (mr < NMI)
          ring[mr % RING] = read_a(abuf, mr / TI, mr % TI);
        else if (NBUF == 3)
          ring[mr % RING] = read_a(b1, 0, mr - NMI);
        if (m == WPOS) load_b(nxt, kb);
        if (!EARLY && m >= A0 && m < A0 + ACH) load_a(ar[m - A0], ka, m - A0);
        // the four dequantization sub-steps of the next slice's B fragment, spread over the
        // slice's TI MFMAs: after every other MFMA at TI = 8, sub-step q after MFMA (q * TI) / 4
        // otherwise
        if constexpr (TI == 8) {
          if ((i & 1) == 0) {
            if (c < 3)
              dq(cur, c + 1, i >> 1, bf[n]);
            else
              dq(nxt, 0, i >> 1, bf[n]);
          }
        } else {
          const int q = dq_sub_at(i, TI);
          if (q >= 0) {
            if (c < 3)
              dq(cur, c + 1, q, bf[n]);
            else
              dq(nxt, 0, q, bf[n]);
          }
        }
        if (c == 3 && i < ACH) {
          *a_dst(NBUF == 3 ? b2 : b1, i) = a_f16(ar[i]);
          if (EARLY) load_a(ar[i], ka2, i);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
    abuf = b1;
  };

  // Prologue: A(0) (and, with three buffers, A(1)) into the first buffers,
  // W(0), the first ring fragments and the slice-0 B fragment; EARLY: A(1)
  // into the chunk registers.
  {
    AR ar1[ACH];
#pragma unroll
    for (int q = 0; q < ACH; ++q) load_a(ar[q], 0, q);
    if constexpr (NBUF == 3) {
#pragma unroll
      for (int q = 0; q < ACH; ++q) load_a(ar1[q], min(1, last), q);
    }
    load_b(wr0, 0);
#pragma unroll
    for (int q = 0; q < ACH; ++q) *a_dst(0, q) = a_f16(ar[q]);
    if constexpr (NBUF == 3) {
#pragma unroll
      for (int q = 0; q < ACH; ++q) *a_dst(1, q) = a_f16(ar1[q]);
    }
    if constexpr (EARLY) {
#pragma unroll
      for (int q = 0; q < ACH; ++q) load_a(ar[q], min(1, last), q);
    }
  }
  __syncthreads();
  if constexpr (NBUF == 3) {
#pragma unroll
    for (int m = 0; m < RD; ++m) ring[m] = read_a(0, m / TI, m % TI);
  }
#pragma unroll
  for (int sub = 0; sub < 4; ++sub) dq(wr0, 0, sub, bf[0]);

  // Pairs of steps with one loop exit (the weight stages alternate); an odd
  // last step runs after the loop.
  int kt = 0;
  for (; kt + 1 < KT; kt += 2) {
    step(kt, wr0, wr1);
    step(kt + 1, wr1, wr0);
  }
  if (kt < KT) step(kt, wr0, wr1);

  store_tile<EPI, TI, TJ, PREB>(d, acc, reinterpret_cast<float*>(smem), wave, lane, m0, cbase, pb0, pb1);
}

// ---------------------------------------------------------------------------
// Small-M kernel: 8 weight rows per workgroup staged in LDS, exact f32 math,
// up to 4 activation rows per pass.
// ---------------------------------------------------------------------------
constexpr int GV_NR = 8;

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

// Output stage shared by the small-M kernels: fin[r * MT + mt] holds the dot
// product of weight row r of the workgroup's segment (SwiGLU: gate rows, then
// the up rows at + V/2) with activation row m0 + mt; bias and epilogue applied.
template <int EPI, int MT, int NR>
__device__ __forceinline__ void gemv_store(const GemmDesc& d, const float* fin, int tid, int r0, int valid, int m0) {
  constexpr int V = NR * MT;
  const int M = d.M, N = d.N;
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
  gemv_store<EPI, MT, GV_NR>(d, fin, tid, r0, valid, m0);
}

// ---------------------------------------------------------------------------
// Medium-M kernel (16 < M < 1024, Q8_0 / Q4_0, K % 64 == 0).  A workgroup owns
// a 32*TI-row x 32*TJ-column output tile (SwiGLU: 16 hidden units in the PAIR
// layout of k_gemm_bf, TJ = 1) and splits K over its waves, KR 64-wide steps
// each; each activation fragment feeds the TJ column groups.  A
// wave issues every load of its K range before the first MFMA: its weight
// row's blocks in the k_gemm_bf lane layout (lane l holds block l/32 of each
// step's 2-block span of row l%32, slice c taking k = 32(l/32) + 8c .. +7) and
// its activation fragments straight from global memory (f32 converted to
// f16), then runs 4*KR*TI MFMAs.  The partial tiles meet in LDS; wave i sums
// 32-row slice i and runs the shared staged epilogue on it.  These shapes are
// latency-bound: one load round trip, a short MFMA chain and one reduction
// replace a K loop per workgroup.
// ---------------------------------------------------------------------------
// B fragment of slice c from a lane's raw dwords of one step (the dequant of
// k_gemm_bf in one piece): exact small integers through the 0x6400 exponent
// trick, the offset removed and d applied in packed f16 (one rounding of d*q).
template <int WT>
__device__ __forceinline__ half8 dq_frag(const uint32_t* r, int c, int h) {
  if constexpr (WT == T0H_F16)  // the lane's 32 weights of the step as they are: slice c is dwords 4c..4c+3
    return __builtin_bit_cast(half8, make_uint4(r[4 * c], r[4 * c + 1], r[4 * c + 2], r[4 * c + 3]));
  const uint32_t qsel = h ? 0x07060504u : 0x05040302u;
  const uint32_t dsel = h ? 0x03020302u : 0x01000100u;
  const int i = WT == T0H_Q8_0 ? 2 * c : 2 * (c & 1);
  uint32_t qa = perm(r[i + 1], r[i], qsel), qb = perm(r[i + 2], r[i + 1], qsel);
  if (WT == T0H_Q4_0) {
    if (c >= 2) {
      qa >>= 4;
      qb >>= 4;
    }
    qa &= 0x0f0f0f0fu;
    qb &= 0x0f0f0f0fu;
  } else {
    qa ^= 0x80808080u;
    qb ^= 0x80808080u;
  }
  const half2v dd = __builtin_bit_cast(half2v, perm(r[0], r[0], dsel));
  const uint32_t t[4] = {perm(0x64646464u, qa, 0x04010400u), perm(0x64646464u, qa, 0x04030402u),
                         perm(0x64646464u, qb, 0x04010400u), perm(0x64646464u, qb, 0x04030402u)};
  const _Float16 o = (_Float16)(WT == T0H_Q8_0 ? 1152.0f : 1032.0f);
  const half2v off = {o, o};
  uint32_t v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(half2v, t[e]) - off) * dd);
  return __builtin_bit_cast(half8, make_uint4(v[0], v[1], v[2], v[3]));
}

template <int WT, bool A32, int EPI, int TI, int KR, int TJ, int RN>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void k_gemm_mid(const GemmDesc d) {
  constexpr bool SWI = EPI == EPI_SWIGLU_F16, F16W = WT == T0H_F16;
  // dwords of a step a lane loads / of a weight row per step (F16: the lane's 32
  // contiguous values; K % 32 == 0, so a lane half of the last step may be past K)
  constexpr int NWD = F16W ? 16 : WT == T0H_Q8_0 ? 9 : 5, SWD = F16W ? 32 : WT == T0H_Q8_0 ? 17 : 9;
  static_assert(!SWI || TJ == 1, "SwiGLU tiles pair gate and up columns in one 32-column group");
  constexpr int W = SWI ? 16 : 32 * TJ;  // output columns per tile
  extern __shared__ __align__(16) float red[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int h = lane >> 5, lc = lane & 31;
  const int M = d.M, N = d.N, K = d.K, KT = (K + 63) / 64;
  auto half_ok = [&](int step) { return !F16W || step * 64 + 32 * h < K; };
  const int strips = (N + W - 1) / W;
  const int tn = blockIdx.x % strips, m0 = (blockIdx.x / strips) * (32 * TI);
  // split RMSNorm consumer: row scales after the partial tiles and the staging
  // (read by the epilogue waves after the barrier below)
  float* const rsc_s = red + nw * TI * TJ * 16 * 64 + TI * 32 * (W + 4);
  if constexpr (RN == 1) row_scales(d, m0, 32 * TI, rsc_s);
  // column group j of the tile: the lane's weight row (rows past N read row 0,
  // activation rows past M read row M-1: never stored)
  const int s0 = wave * KR;
  uint32_t wr[TJ][KR][NWD];
#pragma unroll
  for (int j = 0; j < TJ; ++j) {
    int wrow;
    bool ok;
    if (SWI) {
      const int g = tn * 16 + (lc & 15);
      ok = g < N;
      wrow = lc < 16 ? g : N + g;
    } else {
      wrow = (tn * TJ + j) * 32 + lc;
      ok = wrow < N;
    }
    const uint32_t* wsrc = static_cast<const uint32_t*>(d.w) +
                           (size_t)(ok ? wrow : 0) * (F16W ? K / 2 : (K / 32) * block_bytes(WT) / 4) +
                           h * (F16W ? NWD : NWD - 1);
#pragma unroll
    for (int s = 0; s < KR; ++s)
      if (s0 + s < KT) {
        const uint32_t* src = wsrc + (s0 + s) * SWD;  // NWD contiguous dwords
        if constexpr (F16W) {
          const bool in = half_ok(s0 + s);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4 u = in ? reinterpret_cast<const uint4*>(src)[q] : make_uint4(0, 0, 0, 0);
            wr[j][s][4 * q] = u.x, wr[j][s][4 * q + 1] = u.y, wr[j][s][4 * q + 2] = u.z, wr[j][s][4 * q + 3] = u.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < NWD; ++i) wr[j][s][i] = src[i];
        }
      }
  }
  // The epilogue waves' bias, and for a residual slice its old rows and the
  // producer's norm scales, loaded with the operands (one group of 32 columns,
  // 16-byte stores), so the epilogue starts without a memory round trip.
  constexpr bool PREB = TJ == 1, PREO = TJ == 1 && TI == 1 && EPI == EPI_RESID_F32 && KR <= 4;
  const bool preo = PREO && (d.ldy & 3) == 0 && (N & 3) == 0;
  float pb0 = 0.0f, pb1 = 0.0f;
  float4 pold[PREO ? 4 : 1], pg[PREO ? 4 : 1];
  if (PREB && wave < TI) tile_bias1<EPI>(d, lane, tn * W, pb0, pb1);
  if (PREO && preo && wave == 0) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int idx = t * 64 + lane, row = m0 + idx / 8, col = tn * W + (idx % 8) * 4;
      const bool in = row < M && col < N;
      pold[t] = in ? *reinterpret_cast<const float4*>(static_cast<const float*>(d.y) + (size_t)row * d.ldy + col)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if constexpr (RN == 2) pg[t] = col < N ? *reinterpret_cast<const float4*>(d.norm_g + col)
                                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  half8 af[KR][4][TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) {
    const size_t row = (size_t)min(m0 + 32 * i + lc, M - 1) * d.lda;
#pragma unroll
    for (int s = 0; s < KR; ++s)
      if (s0 + s < KT) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const size_t k = (size_t)(s0 + s) * 64 + 32 * h + 8 * c;
          if (!half_ok(s0 + s)) {
            af[s][c][i] = (half8){};
          } else if (A32) {
            const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + row + k);
            const float4 x0 = src[0], x1 = src[1];
            af[s][c][i] = (half8){(_Float16)x0.x, (_Float16)x0.y, (_Float16)x0.z, (_Float16)x0.w,
                                  (_Float16)x1.x, (_Float16)x1.y, (_Float16)x1.z, (_Float16)x1.w};
          } else {
            af[s][c][i] = *reinterpret_cast<const half8*>(static_cast<const _Float16*>(d.a) + row + k);
          }
        }
      }
  }
  floatx16 acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
#pragma unroll
  for (int s = 0; s < KR; ++s)
    if (s0 + s < KT) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          const half8 b = dq_frag<WT>(wr[j][s], c, h);
#pragma unroll
          for (int i = 0; i < TI; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[s][c][i], b, acc[i][j], 0, 0, 0);
        }
    }
  // partial tiles: [wave][slice][group][quad][lane] float4s (lane-contiguous, no bank conflicts)
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        reinterpret_cast<float4*>(red)[(((wave * TI + i) * TJ + j) * 4 + q) * 64 + lane] =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
  __syncthreads();
  if (wave >= TI) return;
  floatx16 sum[1][TJ];
#pragma unroll
  for (int j = 0; j < TJ; ++j)
#pragma unroll
    for (int e = 0; e < 16; ++e) sum[0][j][e] = 0.0f;
  for (int w = 0; w < nw; ++w)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 v = reinterpret_cast<const float4*>(red)[(((w * TI + wave) * TJ + j) * 4 + q) * 64 + lane];
        sum[0][j][4 * q] += v.x;
        sum[0][j][4 * q + 1] += v.y;
        sum[0][j][4 * q + 2] += v.z;
        sum[0][j][4 * q + 3] += v.w;
      }
  // staging after the partials (other slices may still be reading them)
  float* const stage = red + nw * TI * TJ * 16 * 64;
  if (PREO && preo)
    store_tile<EPI, 1, TJ, PREB, RN, PREO>(d, sum, stage, wave, lane, m0 + 32 * wave, tn * W, pb0, pb1,
                                           rsc_s + 32 * wave, pold, pg);
  else
    store_tile<EPI, 1, TJ, PREB, RN>(d, sum, stage, wave, lane, m0 + 32 * wave, tn * W, pb0, pb1, rsc_s + 32 * wave);
}

// ---------------------------------------------------------------------------
// Small-M kernel for Q8_0 / Q4_0 weights with K % 64 == 0 (M <= MT <= 16).
// 16 lanes per weight row, 16 rows per workgroup (SwiGLU: 8 gate rows and
// their 8 up rows).  A lane owns whole 2-block spans of its row (68 B Q8_0 /
// 36 B Q4_0; a row is K/64 spans, so every span is 4-byte aligned), all of
// them loaded before the first is used.  Arithmetic is f32 with the block scale
// factored out (gguf.rs:116-126, 159-174): a block adds d * sum(q x) for Q8_0 (q
// the signed byte) and d * (sum(u x) - 8 sum(x)) for Q4_0 (u = q + 8 the nibble),
// so a value costs one byte-to-float conversion and one FMA.
// Activations of the MT rows are staged per 1024-wide K tile in LDS as f32
// with each 64-value span padded to 68 floats, so the 16 spans a row group
// reads in one instruction fall in distinct banks (the four row groups of a
// wave read the same addresses: broadcast); for Q4_0 the pad holds the span's
// two block sums of x.  Then a 16-lane DPP reduction and the shared output stage.
// ---------------------------------------------------------------------------
constexpr int GS_NR = 16, GS_TILE = 1024, GS_XS = (GS_TILE / 64) * 68;
// A value the optimizer cannot see into: masked nibble dwords stay whole, so each
// byte becomes one v_cvt_f32_ubyte0..3 instead of a 4-bit field extract per value.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
  asm("" : "+v"(x));
  return x;
}
// The sum of one 32-value block of activations held as a float4 by each of 8 aligned lanes.
__device__ __forceinline__ float block_sum8(float4 v) { return lane_sum8((v.x + v.y) + (v.z + v.w)); }
// The medium-M kernel takes 16 < M < 1024 up to MID_MN_MAX outputs: each of its
// 32-column workgroups reads the whole activation block, so past about 512 x
// 2304 outputs the LDS-staged 128x128 tiles measured faster (M = 512, N = 4096:
// 25 vs 32 us; N = 2304: 24 vs 22 us).
constexpr int MID_M_MAX = 1024;
constexpr long long MID_MN_MAX = 512LL * 2304;

template <int WT, bool A32, int EPI, int MT, int NP>
__global__ __launch_bounds__(256) void k_gemv_s(const GemmDesc d) {
  extern __shared__ __align__(16) float xs[];
  constexpr int DW = WT == T0H_Q8_0 ? 17 : 9;  // dwords per 2-block span
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  const int tid = threadIdx.x, g = tid >> 4, sp = tid & 15;
  const int M = d.M, N = d.N, K = d.K, nsp = K / 64;
  const int r0 = blockIdx.x * (SWI ? GS_NR / 2 : GS_NR);
  const int valid = min(SWI ? GS_NR / 2 : GS_NR, N - r0);
  const int rloc = SWI ? (g & 7) : g;
  // rows past N read row r0 (never stored)
  const int wrow = (rloc < valid ? r0 + rloc : r0) + (SWI && g >= 8 ? N : 0);
  const uint32_t* wr = reinterpret_cast<const uint32_t*>(d.w) + (size_t)wrow * nsp * DW;
  // One row (MT = 1): every K tile of it is staged at once, tile t at xs + t * GS_XS,
  // its loads issued before the weights' so that the stores wait for them alone.
  constexpr bool ALL = MT == 1;
  constexpr int XI = ALL ? NP * GS_TILE / 1024 : 1;  // 16-byte chunks a thread loads
  float4 xv[XI];
  int xk[XI];
  if constexpr (ALL) {
    const int n4 = K / 4;
#pragma unroll
    for (int it = 0; it < XI; ++it) {
      xk[it] = min(tid + 256 * it, n4 - 1) * 4;
      if (A32) {
        xv[it] = *reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + xk[it]);
      } else {
        const half4 hh = *reinterpret_cast<const half4*>(static_cast<const _Float16*>(d.a) + xk[it]);
        xv[it] = make_float4((float)hh[0], (float)hh[1], (float)hh[2], (float)hh[3]);
      }
    }
  }
  // A span is 4-byte aligned: 16-byte loads from it (4 + 1 for Q8_0's 17 dwords, 2 + 1
  // for Q4_0's 9) instead of one load per dword; spans past the row read its last
  // span (no branch: a load under one is waited for inside it) and are not used.
  uint32_t w[NP][DW];
#pragma unroll
  for (int t = 0; t < NP; ++t) {
    const uint32_t* src = wr + min(t * 16 + sp, nsp - 1) * DW;
#pragma unroll
    for (int q = 0; q < DW / 4; ++q) {
      const u32x4_a4 u = *reinterpret_cast<const u32x4_a4*>(src + 4 * q);
      w[t][4 * q] = u.x, w[t][4 * q + 1] = u.y, w[t][4 * q + 2] = u.z, w[t][4 * q + 3] = u.w;
    }
    w[t][DW - 1] = src[DW - 1];
  }
  float acc[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = 0.0f;

  if constexpr (ALL) {
    // (past the row: the last chunk again, written to its own place: the same value)
#pragma unroll
    for (int it = 0; it < XI; ++it) {
      const int k4 = xk[it], t = k4 / GS_TILE, kk = k4 % GS_TILE;
      *reinterpret_cast<float4*>(xs + t * GS_XS + (kk >> 6) * 68 + (kk & 63)) = xv[it];
      if constexpr (WT == T0H_Q4_0) {
        const float bsum = block_sum8(xv[it]);
        if ((tid & 7) == 0 && tid + 256 * it < K / 4) xs[t * GS_XS + (kk >> 6) * 68 + 64 + ((kk >> 5) & 1)] = bsum;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < NP; ++t) {
    const int k0 = t * GS_TILE;
    if (k0 >= K) break;
    const int kn = min(GS_TILE, K - k0);
    if (!ALL && t) __syncthreads();  // the previous tile is consumed
    for (int i = tid; !ALL && i < MT * (kn / 4); i += 256) {
      const int m = i / (kn / 4), k4 = (i % (kn / 4)) * 4;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m < M) {
        if (A32) {
          v = *reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + (size_t)m * d.lda + k0 + k4);
        } else {
          const half4 h = *reinterpret_cast<const half4*>(static_cast<const _Float16*>(d.a) + (size_t)m * d.lda + k0 + k4);
          v = make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
        }
      }
      *reinterpret_cast<float4*>(xs + m * GS_XS + (k4 >> 6) * 68 + (k4 & 63)) = v;
      if constexpr (WT == T0H_Q4_0) {
        const float bsum = block_sum8(v);
        if ((tid & 7) == 0) xs[m * GS_XS + (k4 >> 6) * 68 + 64 + ((k4 >> 5) & 1)] = bsum;
      }
    }
    if (!ALL) __syncthreads();
    const int s = t * 16 + sp;
    if (s < nsp) {
      const uint32_t* r = w[t];
      const float* xr = xs + (ALL ? t * GS_XS : 0) + sp * 68;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        // block h of the span: d at byte (DW*2)*h, quants after it
        const int bo = h * (DW * 2);  // byte offset of the block (34 or 18 per block)
        const uint32_t dw = r[bo >> 2];
        const float dv = (float)__builtin_bit_cast(_Float16, (uint16_t)((bo & 3) ? (dw >> 16) : (dw & 0xffff)));
        float bs[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) bs[m] = 0.0f;
#pragma unroll
        for (int pc = 0; pc < 4; ++pc) {  // 8 consecutive values k = 32h + 8pc .. +7
          float wv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            if (WT == T0H_Q8_0) {
              const int b = bo + 2 + pc * 8 + e;  // byte of value 8pc + e
              wv[e] = (float)(int8_t)(r[b >> 2] >> (8 * (b & 3)));
            } else {
              // quant byte j; high nibbles for values >= 16; the nibbles of a whole
              // dword are masked at once, then each byte converted on its own
              const int j = (pc & 1) * 8 + e, b = bo + 2 + j;
              const uint32_t q = r[b >> 2], nib = opaque_u32((pc >= 2 ? q >> 4 : q) & 0x0f0f0f0fu);
              wv[e] = (float)((nib >> (8 * (b & 3))) & 0xffu);
            }
          }
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            const float4 xa = *reinterpret_cast<const float4*>(xr + m * GS_XS + 32 * h + 8 * pc);
            const float4 xb = *reinterpret_cast<const float4*>(xr + m * GS_XS + 32 * h + 8 * pc + 4);
            float a = bs[m];
            a = fmaf(wv[0], xa.x, a); a = fmaf(wv[1], xa.y, a); a = fmaf(wv[2], xa.z, a); a = fmaf(wv[3], xa.w, a);
            a = fmaf(wv[4], xb.x, a); a = fmaf(wv[5], xb.y, a); a = fmaf(wv[6], xb.z, a); a = fmaf(wv[7], xb.w, a);
            bs[m] = a;
          }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          if (WT == T0H_Q8_0)
            acc[m] = fmaf(dv, bs[m], acc[m]);
          else
            acc[m] = fmaf(dv, fmaf(-8.0f, xr[m * GS_XS + 64 + h], bs[m]), acc[m]);
        }
      }
    }
  }
#pragma unroll
  for (int m = 0; m < MT; ++m) acc[m] = lane_sum16(acc[m]);
  __syncthreads();  // activations no longer needed: reuse LDS for the row sums
  float* fin = xs;
  if (sp == 0) {
#pragma unroll
    for (int m = 0; m < MT; ++m) fin[g * MT + m] = acc[m];
  }
  __syncthreads();
  gemv_store<EPI, MT, GS_NR>(d, fin, tid, r0, valid, 0);
}

// ---------------------------------------------------------------------------
// M = 1 kernel for long Q8_0 / Q4_0 rows: K = 4096 SP (SP = 1, 2), 64 SP
// two-block spans a row.  Lane l of a wave owns spans l + 64 j of every row the
// wave takes, so the activations of those spans are read from LDS into its
// registers once and serve all of its rows: a row then costs one coalesced load
// of 64 x 36 (Q4_0) or 68 (Q8_0) bytes a span column and, a value, one
// byte-to-float conversion and one FMA, with the block scale factored out as in
// k_gemv_s.  Q4_0 nibbles: the low ones masked to bytes (u), the high ones kept
// in place (16 u, an exact power-of-two scale undone once a block).  A wave
// takes R rows, all loaded before the first is used; the four waves' row
// partials meet in LDS and 8 lanes finish each row.
// ---------------------------------------------------------------------------
// Rows a wave takes: 4 (16 a workgroup, so K = 4096, N = 16384 fills 1024 workgroups),
// 2 when the activations take 128 registers (K = 8192).
constexpr int gw_rows(int sp) { return sp == 1 ? 4 : 2; }

template <int WT, bool A32, int EPI, int SP>
__global__ __launch_bounds__(256) void k_gemv_w(const GemmDesc d) {
  extern __shared__ __align__(16) float xs[];  // 64 SP spans of 68 floats, then the row partials
  constexpr int DW = WT == T0H_Q8_0 ? 17 : 9;  // dwords per span
  constexpr int R = gw_rows(SP), NRW = 4 * R;
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  constexpr int PER = SWI ? NRW / 2 : NRW;  // output columns of a workgroup
  constexpr int XI = SP * 4;                // 16-byte activation chunks a thread stages
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int N = d.N, nsp = 64 * SP;
  const int r0 = blockIdx.x * PER;
  const int valid = min(PER, N - r0);
  float4 xv[XI];
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const int k = (tid + 256 * it) * 4;
    if (A32) {
      xv[it] = *reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + k);
    } else {
      const half4 hh = *reinterpret_cast<const half4*>(static_cast<const _Float16*>(d.a) + k);
      xv[it] = make_float4((float)hh[0], (float)hh[1], (float)hh[2], (float)hh[3]);
    }
  }
  // local row w R + i: output column c (SwiGLU: gate rows, then their up rows);
  // columns past N read the workgroup's first row (never stored)
  uint32_t w[R][SP][DW];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int lr = wave * R + i, c = SWI && lr >= PER ? lr - PER : lr;
    const int row = (c < valid ? r0 + c : r0) + (SWI && lr >= PER ? N : 0);
    const uint32_t* wr = reinterpret_cast<const uint32_t*>(d.w) + (size_t)row * nsp * DW;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      const uint32_t* src = wr + (lane + 64 * j) * DW;
#pragma unroll
      for (int q = 0; q < DW / 4; ++q) {
        const u32x4_a4 u = *reinterpret_cast<const u32x4_a4*>(src + 4 * q);
        w[i][j][4 * q] = u.x, w[i][j][4 * q + 1] = u.y, w[i][j][4 * q + 2] = u.z, w[i][j][4 * q + 3] = u.w;
      }
      w[i][j][DW - 1] = src[DW - 1];
    }
  }
#pragma unroll
  for (int it = 0; it < XI; ++it) {
    const int k = (tid + 256 * it) * 4;
    *reinterpret_cast<float4*>(xs + (k >> 6) * 68 + (k & 63)) = xv[it];
  }
  __syncthreads();
  float x[SP][64];
#pragma unroll
  for (int j = 0; j < SP; ++j) {
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const float4 v = *reinterpret_cast<const float4*>(xs + (lane + 64 * j) * 68 + 4 * c);
      x[j][4 * c] = v.x, x[j][4 * c + 1] = v.y, x[j][4 * c + 2] = v.z, x[j][4 * c + 3] = v.w;
    }
  }
  float sx[SP][2];  // Q4_0: the block sums of x
#pragma unroll
  for (int j = 0; j < SP; ++j) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float a = 0.0f;
#pragma unroll
      for (int v = 0; v < 32; ++v) a += x[j][32 * h + v];
      sx[j][h] = WT == T0H_Q4_0 ? a : 0.0f;
    }
  }
  float* part = xs + 64 * SP * 68;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < SP; ++j) {
      const uint32_t* r = w[i][j];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int bo = h * (DW * 2);  // byte offset of block h (34 or 18 bytes a block)
        const uint32_t dw = r[bo >> 2];
        const float dv = (float)__builtin_bit_cast(_Float16, (uint16_t)((bo & 3) ? (dw >> 16) : (dw & 0xffff)));
        if (WT == T0H_Q8_0) {
          float b0 = 0.0f, b1 = 0.0f;
#pragma unroll
          for (int v = 0; v < 32; v += 2) {
            const int b = bo + 2 + v, c = b + 1;
            b0 = fmaf((float)(int8_t)(r[b >> 2] >> (8 * (b & 3))), x[j][32 * h + v], b0);
            b1 = fmaf((float)(int8_t)(r[c >> 2] >> (8 * (c & 3))), x[j][32 * h + v + 1], b1);
          }
          acc = fmaf(dv, b0 + b1, acc);
        } else {
          float bl = 0.0f, bh = 0.0f;  // low nibbles (values 0..15), high nibbles x 16 (16..31)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int b = bo + 2 + v;
            const uint32_t lo = opaque_u32(r[b >> 2] & 0x0f0f0f0fu), hi = opaque_u32(r[b >> 2] & 0xf0f0f0f0u);
            bl = fmaf((float)((lo >> (8 * (b & 3))) & 0xffu), x[j][32 * h + v], bl);
            bh = fmaf((float)((hi >> (8 * (b & 3))) & 0xffu), x[j][32 * h + 16 + v], bh);
          }
          acc = fmaf(dv, fmaf(-8.0f, sx[j][h], fmaf(bh, 0.0625f, bl)), acc);
        }
      }
    }
    part[(wave * R + i) * 64 + lane] = acc;
  }
  __syncthreads();
  // row t / 8 summed by 8 lanes (aligned groups: all active); the activations are
  // no longer read, so the row sums reuse their LDS
  float rsum = 0.0f;
  if (tid < NRW * 8) {
    const float4 a = *reinterpret_cast<const float4*>(part + tid * 8);
    const float4 b = *reinterpret_cast<const float4*>(part + tid * 8 + 4);
    rsum = lane_sum8(((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)));
  }
  if (tid < NRW * 8 && (tid & 7) == 0) xs[tid >> 3] = rsum;
  __syncthreads();
  gemv_store<EPI, 1, NRW>(d, xs, tid, r0, valid, 0);
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

template <int WT, bool A32, int EPI, bool K64, int TI, int TJ>
void run_gemm(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  using C = Tile<TI, TJ>;
  const int hb = EPI == EPI_SWIGLU_F16 ? C::BN / 2 : C::BN;
  const int tiles_n = (d.N + hb - 1) / hb;
  const int tiles_m = (d.M + C::BM - 1) / C::BM;
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm<WT, A32, EPI, K64, TI, TJ>), lds_set);
  hipLaunchKernelGGL((k_gemm<WT, A32, EPI, K64, TI, TJ>), dim3(tiles_m * tiles_n), dim3(256), C::LDS, s, d);
  check_hip(hipGetLastError(), "k_gemm launch");
}

// Tile choice.  tile: 0 = by shape, 1 = 128x128, 2 = 256x128, 3 = 256x256.
// The larger tiles are built for f16 activations with 4-byte-aligned weight
// rows (K % 64 == 0), the shapes of the model's layers.
// The DMA kernel needs an even number of 64-wide K steps and output rows
// that take 16-byte (f32) / 8-byte (f16) vector stores.
bool dma_ok(const GemmDesc& d) { return d.K % 128 == 0 && d.N % 4 == 0 && d.ldy % 4 == 0; }

template <int WT, int EPI>
void run_gemm_dma(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  const int hb = EPI == EPI_SWIGLU_F16 ? DM_BN / 2 : DM_BN;
  const int tiles_n = (d.N + hb - 1) / hb;
  const int tiles_m = (d.M + DM_BM - 1) / DM_BM;
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm_dma<WT, EPI>), lds_set);
  hipLaunchKernelGGL((k_gemm_dma<WT, EPI>), dim3(tiles_m * tiles_n), dim3(256), DM_LDS, s, d);
  check_hip(hipGetLastError(), "k_gemm_dma launch");
}

template <int WT, int EPI, int NWV, bool A32 = false, int BM = BF_BM>
void run_gemm_bf(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  using C = BfCfg<NWV, BM>;
  const int hb = EPI == EPI_SWIGLU_F16 ? C::BN / 2 : C::BN;
  const int n_tiles = ((d.N + hb - 1) / hb) * ((d.M + BM - 1) / BM);
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm_bf<WT, EPI, NWV, A32, BM>), lds_set);
  hipLaunchKernelGGL((k_gemm_bf<WT, EPI, NWV, A32, BM>), dim3(n_tiles), dim3(64 * NWV), C::LDS, s, d);
  check_hip(hipGetLastError(), "k_gemm_bf launch");
}

template <int WT, bool A32, int EPI, bool K64>
void run_gemm_tiled(const GemmDesc& d, int tile, hipStream_t s) {
  // By shape (tile 0).  Measured at the config-4 layer shapes (M = 50,688,
  // Q4_0, us; register-operand 256x128 at two workgroups per CU / 256x256 /
  // 128x128): SwiGLU 360 / 363 / 430, QKV 250 / 245 / 290, wO 97 / 103 / 107,
  // w2 224 / 232 / 238 (standalone).  Inside the forward QKV measured 213.5 us
  // on the 256x128 kernel against 217.5 on the 256x256 one, so it takes the
  // 256x128 kernel too.  The DMA and plain 256x256 tiles lose at every shape.
  // 192- and 128-row tiles (7, 8), which would fill the last round of the
  // N = 768 launches better (1,188 tiles are 2.32 rounds of 512 slots), measured
  // slower inside the config-4 forward at every layer GEMM (Q4_0 step 12.80 ->
  // 13.24 / 13.73 ms; Q8_0 13.47 -> 14.12 / 14.81): each weight fragment then
  // feeds 6 or 4 MFMAs instead of 8.
  // Below ~1024 rows a 256-row tile is mostly padding.
  if (tile == 0) {
    tile = 1;
    if constexpr (!A32 && K64 && WT != T0H_F16)
      if (d.M >= 1024) tile = 6;
    // f32 activations (f32 stores only): the 256x256 register-operand kernel
    // converts them while staging
    if constexpr (A32 && K64 && WT != T0H_F16 && EPI == EPI_STORE_F32)
      if (d.M >= 1024) return run_gemm_bf<WT, EPI, 8, true>(d, s);
  }
  if constexpr (!A32 && K64 && WT != T0H_F16) {
    if (tile == 4 && dma_ok(d)) return run_gemm_dma<WT, EPI>(d, s);
    if (tile == 5) return run_gemm_bf<WT, EPI, 8>(d, s);
    if (tile == 6) return run_gemm_bf<WT, EPI, 4>(d, s);
    if (tile == 7) return run_gemm_bf<WT, EPI, 4, false, 192>(d, s);
    if (tile == 8) return run_gemm_bf<WT, EPI, 4, false, 128>(d, s);
  }
  if constexpr (!A32 && K64) {
    if (tile == 3 || tile == 4) return run_gemm<WT, A32, EPI, K64, 4, 4>(d, s);
    if (tile == 2) return run_gemm<WT, A32, EPI, K64, 4, 2>(d, s);
  }
  run_gemm<WT, A32, EPI, K64, 2, 2>(d, s);
}

// ---------------------------------------------------------------------------
// Small-M kernel for 2 <= M <= 16 rows (any weight type, K % 32 == 0): exact
// f32 products on v_mfma_f32_16x16x4f32.  A workgroup owns NB groups of 16 weight
// rows (SwiGLU: 8 gate rows and their 8 up rows) and splits K over MF_WAVES waves,
// block kb going to wave kb % MF_WAVES.  In a 32-value block, lane (j, c) =
// (lane % 16, lane / 16) dequantizes values 8c .. 8c+7 of weight row j exactly
// (f32(d) * q: an 11-bit scale times an integer of at most 8 bits; f16 weights
// convert exactly) and holds activations 8c .. 8c+7 of row j; MFMA s of the
// block takes value 8c + s from every lane, so each product of the block is
// summed once.  The waves' 16x16 partial tiles are summed in LDS in wave order
// and written by one thread per output (bias, ReLU, residual add or SwiGLU).
// The weights are read with 2-byte loads (Q8_0 / Q4_0 blocks are 2-byte
// aligned), never past a block.
// ---------------------------------------------------------------------------
constexpr int MF_WAVES = 8;  // waves per workgroup

// NB groups of 16 weight columns a workgroup (4 for wide matrices: every activation value a lane
// loads then feeds 4 groups' MFMAs instead of one); CH blocks per load batch.
template <int WT, bool A32, int EPI, int NB>
__global__ __launch_bounds__(64 * MF_WAVES) void k_gemv_mf(const GemmDesc d) {
  constexpr int CH = NB == 1 ? 4 : 2;
  __shared__ float red[NB][MF_WAVES][16][17];
  constexpr bool SWI = EPI == EPI_SWIGLU_F16;
  constexpr int GC = SWI ? 8 : 16;  // output columns of a group
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, j = lane & 15, c = lane >> 4;
  const int M = d.M, N = d.N, K = d.K, KB = K / 32;
  const int c0 = blockIdx.x * GC * NB;  // first output column (SwiGLU: hidden unit)
  const size_t rowb = WT == T0H_F16 ? (size_t)K * 2 : (size_t)KB * block_bytes(WT);
  const uint8_t* wr[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    int wrow;
    if (SWI) {
      const int u = min(c0 + nb * GC + (j & 7), N - 1);
      wrow = j < 8 ? u : N + u;
    } else {
      wrow = min(c0 + nb * GC + j, N - 1);  // rows past N are computed, never stored
    }
    wr[nb] = static_cast<const uint8_t*>(d.w) + (size_t)wrow * rowb;
  }
  const bool arow = j < M;
  const size_t aoff = (size_t)(arow ? j : 0) * d.lda + 8 * c;

  // one block's operands for this lane: 8 weights (raw) of each group and 8 activations
  struct Op {
    uint32_t w[NB][4];  // Q8_0 / Q4_0: 4 x 2 bytes (+ the scale in sc); f16: 8 halves
    uint32_t sc[NB];
    uint32_t a[A32 ? 8 : 4];
  };
  auto load = [&](int kb, Op& o) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (WT == T0H_F16) {
        const uint4 v = *reinterpret_cast<const uint4*>(wr[nb] + (size_t)(kb * 32 + 8 * c) * 2);
        o.w[nb][0] = v.x, o.w[nb][1] = v.y, o.w[nb][2] = v.z, o.w[nb][3] = v.w;
        o.sc[nb] = 0;
      } else {
        const uint8_t* b = wr[nb] + (size_t)kb * block_bytes(WT);
        const uint16_t* q = reinterpret_cast<const uint16_t*>(b + 2 + (WT == T0H_Q8_0 ? 8 * c : 8 * (c & 1)));
#pragma unroll
        for (int e = 0; e < 4; ++e) o.w[nb][e] = q[e];
        o.sc[nb] = *reinterpret_cast<const uint16_t*>(b);
      }
    }
    if (arow) {
      if constexpr (A32) {
        const float4* x = reinterpret_cast<const float4*>(static_cast<const float*>(d.a) + aoff + (size_t)kb * 32);
        const float4 x0 = x[0], x1 = x[1];
        o.a[0] = __float_as_uint(x0.x), o.a[1] = __float_as_uint(x0.y), o.a[2] = __float_as_uint(x0.z);
        o.a[3] = __float_as_uint(x0.w), o.a[4] = __float_as_uint(x1.x), o.a[5] = __float_as_uint(x1.y);
        o.a[6] = __float_as_uint(x1.z), o.a[7] = __float_as_uint(x1.w);
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const _Float16*>(d.a) + aoff + (size_t)kb * 32);
        o.a[0] = v.x, o.a[1] = v.y, o.a[2] = v.z, o.a[3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < (A32 ? 8 : 4); ++e) o.a[e] = 0;
    }
  };
  auto weight = [&](const Op& o, int nb, int s) -> float {
    if constexpr (WT == T0H_F16) {
      return (float)__builtin_bit_cast(half2v, o.w[nb][s >> 1])[s & 1];
    } else {
      const float dd = (float)__builtin_bit_cast(_Float16, (uint16_t)o.sc[nb]);
      const uint32_t byte = (o.w[nb][s >> 1] >> (8 * (s & 1))) & 0xffu;
      if constexpr (WT == T0H_Q8_0) return dd * (float)(int8_t)byte;
      const uint32_t nib = c >= 2 ? byte >> 4 : byte & 15u;
      return dd * (float)((int)nib - 8);
    }
  };
  auto act = [&](const Op& o, int s) -> float {
    if constexpr (A32) return __uint_as_float(o.a[s]);
    return (float)__builtin_bit_cast(half2v, o.a[s >> 1])[s & 1];
  };

  floatx4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  // batches of CH blocks, the next batch's loads issued before this one's MFMAs
  Op ops[2][CH];
  auto load_batch = [&](int kb0, Op(&o)[CH]) {
#pragma unroll
    for (int q = 0; q < CH; ++q)
      if (kb0 + q * MF_WAVES < KB) load(kb0 + q * MF_WAVES, o[q]);
  };
  auto run_batch = [&](int kb0, const Op(&o)[CH]) {
#pragma unroll
    for (int q = 0; q < CH; ++q)
      if (kb0 + q * MF_WAVES < KB) {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float av = act(o[q], s);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            acc[nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, weight(o[q], nb, s), acc[nb], 0, 0, 0);
        }
      }
  };
  constexpr int STEP = MF_WAVES * CH;
  load_batch(wave, ops[0]);
  // the output threads' bias (and old residual value), loaded with the first batch
  const int m = tid >> 4, jj = tid & 15;
  float pb[NB], pb2[NB], py[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = c0 + nb * GC + jj;
    const bool outp = tid < 256 && m < M && (SWI ? jj < 8 : true) && col < N;
    pb[nb] = 0.0f, pb2[nb] = 0.0f, py[nb] = 0.0f;
    if (outp) {
      if (d.bias) {
        pb[nb] = d.bias[col];
        if constexpr (SWI) pb2[nb] = d.bias[N + col];
      }
      if constexpr (EPI == EPI_RESID_F32) py[nb] = static_cast<const float*>(d.y)[(size_t)m * d.ldy + col];
    }
  }
  int kb0 = wave;
  for (; kb0 + STEP < KB; kb0 += 2 * STEP) {  // pairs of batches: the buffers alternate
    load_batch(kb0 + STEP, ops[1]);
    run_batch(kb0, ops[0]);
    if (kb0 + 2 * STEP < KB) load_batch(kb0 + 2 * STEP, ops[0]);
    run_batch(kb0 + STEP, ops[1]);
  }
  if (kb0 < KB) run_batch(kb0, ops[0]);
  // D layout: lane l, register r -> row 4 (l / 16) + r, column l % 16
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[nb][wave][4 * c + r][j] = acc[nb][r];
  }
  __syncthreads();
  if (tid >= 256 || m >= M || (SWI && jj >= 8)) return;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = c0 + nb * GC + jj;
    if (col >= N) break;
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < MF_WAVES; ++w) v += red[nb][w][m][jj];
    if constexpr (SWI) {
      float up = 0.0f;
#pragma unroll
      for (int w = 0; w < MF_WAVES; ++w) up += red[nb][w][m][jj + 8];
      const float g = v + pb[nb], uu = up + pb2[nb];
      static_cast<_Float16*>(d.y)[(size_t)m * d.ldy + col] = (_Float16)(silu(g) * uu);
    } else {
      v += pb[nb];
      if (d.relu) v = fmaxf(v, 0.0f);
      const size_t o = (size_t)m * d.ldy + col;
      if constexpr (EPI == EPI_RESID_F32) {
        static_cast<float*>(d.y)[o] = py[nb] + v;
      } else if constexpr (EPI == EPI_STORE_F32) {
        static_cast<float*>(d.y)[o] = v;
      } else {
        static_cast<_Float16*>(d.y)[o] = (_Float16)v;
      }
    }
  }
}

template <int WT, bool A32, int EPI, int NB>
void launch_gemv_mf(const GemmDesc& d, hipStream_t s) {
  const int per = (EPI == EPI_SWIGLU_F16 ? 8 : 16) * NB;
  hipLaunchKernelGGL((k_gemv_mf<WT, A32, EPI, NB>), dim3((d.N + per - 1) / per), dim3(64 * MF_WAVES), 0, s, d);
  check_hip(hipGetLastError(), "k_gemv_mf launch");
}

// Four column groups a workgroup once that still leaves a workgroup per CU (N >= 16384
// columns; 8192 SwiGLU units), two from half that; one below.
template <int WT, bool A32, int EPI>
void run_gemv_mf(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  const int groups = (d.N + (EPI == EPI_SWIGLU_F16 ? 7 : 15)) / (EPI == EPI_SWIGLU_F16 ? 8 : 16);
  if (groups >= 4 * 256) return launch_gemv_mf<WT, A32, EPI, 4>(d, s);
  if (groups >= 2 * 256) return launch_gemv_mf<WT, A32, EPI, 2>(d, s);
  launch_gemv_mf<WT, A32, EPI, 1>(d, s);
}

// The f32-MFMA small-M kernel's operand loads: 16-byte activation chunks and,
// for f16 weights, 16-byte weight chunks; no table row add.
bool gemv_mf_ok(const GemmDesc& d) {
  const bool a16 = (reinterpret_cast<uintptr_t>(d.a) & 15) == 0 && d.lda % (d.a_f32 ? 4 : 8) == 0;
  const bool w16 = d.wtype != T0H_F16 || (reinterpret_cast<uintptr_t>(d.w) & 15) == 0;
  const bool w2 = (reinterpret_cast<uintptr_t>(d.w) & 1) == 0;
  return d.M >= 2 && d.M <= 16 && d.K % 32 == 0 && a16 && w16 && w2 && !d.row_add;
}

template <int WT, bool A32, int EPI, int MT>
void run_gemv(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  const size_t rb = WT == T0H_F16 ? (size_t)d.K * 2 : (size_t)(d.K / 32) * block_bytes(WT);
  const size_t lds = std::max<size_t>(GV_NR * rb, 5 * GV_NR * MT * sizeof(float));
  const int seg_rows = EPI == EPI_SWIGLU_F16 ? GV_NR / 2 : GV_NR;
  const int gx = (d.N + seg_rows - 1) / seg_rows, gy = (d.M + MT - 1) / MT;
  if (lds > 160 * 1024) throw Error(T0H_ERR_UNSUPPORTED, "gemv: K too large for the LDS row stage");
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemv<WT, A32, EPI, MT>), lds_set);
  hipLaunchKernelGGL((k_gemv<WT, A32, EPI, MT>), dim3(gx, gy), dim3(256), lds, s, d);
  check_hip(hipGetLastError(), "k_gemv launch");
}

template <int WT, bool A32, int EPI, int MT, int NP>
void run_gemv_s(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  const size_t lds = (size_t)(MT == 1 ? NP : MT) * GS_XS * sizeof(float);
  const int per = EPI == EPI_SWIGLU_F16 ? GS_NR / 2 : GS_NR;
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemv_s<WT, A32, EPI, MT, NP>), lds_set);
  hipLaunchKernelGGL((k_gemv_s<WT, A32, EPI, MT, NP>), dim3((d.N + per - 1) / per), dim3(256), lds, s, d);
  check_hip(hipGetLastError(), "k_gemv_s launch");
}

template <int WT, bool A32, int EPI, int SP>
void run_gemv_w(const GemmDesc& d, hipStream_t s) {
  if (d.row_ssq || d.norm_out) throw Error(T0H_ERR_HIP, "internal: split RMSNorm on a kernel without it");
  if (d.M != 1 || d.K != 4096 * SP) throw Error(T0H_ERR_HIP, "internal: gemv_w shape");
  constexpr int NRW = 4 * gw_rows(SP), per = EPI == EPI_SWIGLU_F16 ? NRW / 2 : NRW;
  const size_t lds = (size_t)(64 * SP * 68 + NRW * 64) * sizeof(float);
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemv_w<WT, A32, EPI, SP>), lds_set);
  hipLaunchKernelGGL((k_gemv_w<WT, A32, EPI, SP>), dim3((d.N + per - 1) / per), dim3(256), lds, s, d);
  check_hip(hipGetLastError(), "k_gemv_w launch");
}

template <int WT, bool A32, int EPI, int MT>
void dispatch_gemv_s(const GemmDesc& d, hipStream_t s) {
  if (d.K <= GS_TILE)
    run_gemv_s<WT, A32, EPI, MT, 1>(d, s);
  else if (d.K <= 2 * GS_TILE)
    run_gemv_s<WT, A32, EPI, MT, 2>(d, s);
  else
    run_gemv_s<WT, A32, EPI, MT, 4>(d, s);
}

template <int WT, bool A32, int EPI>
void dispatch_gemv(const GemmDesc& d, hipStream_t s) {
  // 2..16 rows: exact f32 on the f32 MFMA (the LDS-staged f32 kernels below redo
  // every activation row per weight row: M = 16 took 10 us at K = 768, N = 2304)
  if (gemv_mf_ok(d)) return run_gemv_mf<WT, A32, EPI>(d, s);
  if constexpr (WT != T0H_F16) {
    if (d.M == 1 && d.K == 4096) return run_gemv_w<WT, A32, EPI, 1>(d, s);
    if (d.M == 1 && d.K == 8192) return run_gemv_w<WT, A32, EPI, 2>(d, s);
    if (d.M <= 16 && d.K % 64 == 0 && d.K <= 4 * GS_TILE) {
      if (d.M == 1) return dispatch_gemv_s<WT, A32, EPI, 1>(d, s);
      if (d.M <= 4) return dispatch_gemv_s<WT, A32, EPI, 4>(d, s);
      return dispatch_gemv_s<WT, A32, EPI, 16>(d, s);
    }
  }
  if (d.M == 1)
    run_gemv<WT, A32, EPI, 1>(d, s);
  else if (d.M == 2)
    run_gemv<WT, A32, EPI, 2>(d, s);
  else
    run_gemv<WT, A32, EPI, 4>(d, s);
}

// Waves of KR steps over K (at most 8 per workgroup, two per SIMD, so a wave
// may hold its KR steps of operands: up to 256 registers); lds: the partial
// tiles and the epilogue staging of TI waves.
template <int WT, bool A32, int EPI, int TI, int KR, int TJ, int RN>
void launch_gemm_mid(const GemmDesc& d, hipStream_t s) {
  // at least one wave per 32-row slice: slice i is summed and stored by wave i
  const int KT = d.K / 64, nw = std::max(TI, (KT + KR - 1) / KR);
  if (nw > 8) throw Error(T0H_ERR_UNSUPPORTED, "gemm: K too large for the medium-M kernel");
  const int W = EPI == EPI_SWIGLU_F16 ? 16 : 32 * TJ;
  const size_t lds = (size_t)nw * TI * TJ * 16 * 64 * 4 + (size_t)TI * 32 * (W + 4) * 4 + (RN == 1 ? TI * 32 * 4 : 0);
  const int strips = (d.N + W - 1) / W, mt = (d.M + 32 * TI - 1) / (32 * TI);
  static std::atomic<uint64_t> lds_set{0};  // per instantiation
  allow_dynamic_lds(reinterpret_cast<const void*>(&k_gemm_mid<WT, A32, EPI, TI, KR, TJ, RN>), lds_set);
  hipLaunchKernelGGL((k_gemm_mid<WT, A32, EPI, TI, KR, TJ, RN>), dim3(strips * mt), dim3(64 * nw), lds, s, d);
  check_hip(hipGetLastError(), "k_gemm_mid launch");
}

// The split RMSNorm roles (GemmDesc) are instantiations of their own: a consumer
// is an f16-store or SwiGLU GEMM, a producer a residual one.
template <int WT, bool A32, int EPI, int TI, int KR, int TJ = 1>
void run_gemm_mid(const GemmDesc& d, hipStream_t s) {
  if constexpr (EPI == EPI_RESID_F32) {
    if (d.row_ssq) throw Error(T0H_ERR_HIP, "internal: a residual GEMM cannot consume the split RMSNorm");
    if (d.norm_out) {
      if (d.N % 32 || d.ldy % 4) throw Error(T0H_ERR_HIP, "internal: split RMSNorm producer needs N % 32 == 0");
      return launch_gemm_mid<WT, A32, EPI, TI, KR, TJ, 2>(d, s);
    }
  } else {
    if (d.norm_out) throw Error(T0H_ERR_HIP, "internal: only a residual GEMM produces the split RMSNorm");
    if constexpr (!A32 && (EPI == EPI_STORE_F16 || EPI == EPI_SWIGLU_F16))
      if (d.row_ssq) return launch_gemm_mid<WT, A32, EPI, TI, KR, TJ, 1>(d, s);
    if (d.row_ssq) throw Error(T0H_ERR_HIP, "internal: split RMSNorm consumer on an unsupported epilogue");
  }
  launch_gemm_mid<WT, A32, EPI, TI, KR, TJ, 0>(d, s);
}

// Compute units of the current device (the round size of a launch).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    hipDeviceProp_t prop;
    check_hip(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    cus[dev] = std::max(1, prop.multiProcessorCount);
  }
  return cus[dev];
}

// Shapes the medium-M kernel takes: K % 64 == 0 and K <= 4096 (f16 activations)
// or 2048 (f32); 32-row tiles for f32 activations or M < 256, else 64.  From
// 256 rows (and not SwiGLU) a workgroup may cover four or two 32-column groups
// (two past K = 1024), so the activation block is read by a quarter or half as
// many workgroups, when that still fills about one round of the CUs.
bool mid_ok(const GemmDesc& d) {
  if (d.wtype == T0H_F16) return d.K % 32 == 0 && d.K <= 2048;  // (16-dword spans: at most 4 steps a wave)
  return d.K % 64 == 0 && d.K <= (d.a_f32 ? 2048 : 4096);
}

// Workgroups of a TJ-group launch with 32-row tiles, and whether they fill
// between three quarters of a round and one round of the device's CUs (the
// LDS of the partial tiles bounds the workgroups per CU).
bool mid_groups_fit(const GemmDesc& d, int tj, int kr) {
  const int KT = (d.K + 63) / 64, nw = std::max(1, (KT + kr - 1) / kr), cus = device_cus();
  const long long wgs = (long long)((d.N + 32 * tj - 1) / (32 * tj)) * ((d.M + 31) / 32);
  const size_t lds = (size_t)nw * tj * 16 * 64 * 4 + (size_t)32 * (32 * tj + 4) * 4;
  const long long per_cu = std::max<long long>(1, (long long)(160 * 1024 / lds));
  return nw <= 8 && wgs * 4 >= 3LL * cus && wgs <= per_cu * cus;
}

template <int WT, bool A32, int EPI>
void dispatch_mid(const GemmDesc& d, hipStream_t s) {
  const int KT = (d.K + 63) / 64;
  if constexpr (EPI != EPI_SWIGLU_F16 && WT != T0H_F16) {  // (F16 spans are 16 dwords: one column group)
    if (d.M >= 256 && KT <= 32) {
      const int kr = KT <= 16 ? 2 : 4;
      if (kr == 2 && mid_groups_fit(d, 4, 2)) return run_gemm_mid<WT, A32, EPI, 1, 2, 4>(d, s);
      if (mid_groups_fit(d, 2, kr)) {  // (4 groups x 4 steps of Q8_0 spans spill)
        if (kr == 2) return run_gemm_mid<WT, A32, EPI, 1, 2, 2>(d, s);
        return run_gemm_mid<WT, A32, EPI, 1, 4, 2>(d, s);
      }
    }
  }
  // 32-row tiles below 256 rows: more workgroups, each with a shorter operand
  // set (measured at M = 66 / 198, Q8_0: w2 14.0 -> 9.9 / 14.2 -> 10.2 us, QKV
  // 6.9 -> 5.9, wO 6.8 -> 5.9, SwiGLU 7.2 -> 6.8 / 11.6 -> 10.7 us)
  // (F16 spans hold twice the registers: 64-row tiles only with two steps a wave)
  if (A32 || d.M < 256 || KT > 32 || (WT == T0H_F16 && KT > 16)) {
    if (KT <= 16) return run_gemm_mid<WT, A32, EPI, 1, 2>(d, s);
    if (KT <= 32) return run_gemm_mid<WT, A32, EPI, 1, 4>(d, s);
    if constexpr (!A32 && WT != T0H_F16) return run_gemm_mid<WT, A32, EPI, 1, 8>(d, s);
  } else {
    if (KT <= 16) return run_gemm_mid<WT, A32, EPI, 2, 2>(d, s);
    if constexpr (WT != T0H_F16) return run_gemm_mid<WT, A32, EPI, 2, 4>(d, s);
  }
  throw Error(T0H_ERR_UNSUPPORTED, "gemm: shape outside the medium-M kernel");
}

template <int WT, bool A32, int EPI>
void dispatch_w(const GemmDesc& d, int force, hipStream_t s) {
  // medium M (force 0) or FORCE_MID
  const bool mid = force == 0 && d.M > 16 && d.M < MID_M_MAX && (long long)d.M * d.N <= MID_MN_MAX;
  if ((force == FORCE_MID || mid) && mid_ok(d)) return dispatch_mid<WT, A32, EPI>(d, s);
  const bool mfma = force == 1 || (force >= 3 && force != FORCE_MID) || (force == 0 && d.M > 16);
  if (mfma) {
    const int tile = force >= 3 ? force - 2 : 0;
    if (d.K % 64 == 0)
      run_gemm_tiled<WT, A32, EPI, true>(d, tile, s);
    else
      run_gemm_tiled<WT, A32, EPI, false>(d, tile, s);
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

// Mirrors the automatic choice (force 0) of dispatch_w: only the medium-M kernel
// (f16 activations, 16 < M < 1024 up to MID_MN_MAX outputs, the K of mid_ok) has
// the split RMSNorm epilogues.
namespace {
bool mid_auto(const GemmDesc& d) {
  return !d.a_f32 && d.M > 16 && d.M < MID_M_MAX && (long long)d.M * d.N <= MID_MN_MAX && mid_ok(d);
}
}  // namespace
bool rownorm_producer_ok(const GemmDesc& d) {
  return d.epi == EPI_RESID_F32 && mid_auto(d) && d.N % 32 == 0 && d.ldy % 4 == 0 && !d.row_add;
}
bool rownorm_consumer_ok(const GemmDesc& d) {
  if (d.epi != EPI_STORE_F16 && d.epi != EPI_SWIGLU_F16) return false;
  if (d.ssq_parts % 4 || d.ssq_parts > RN_MAX_PARTS) return false;
  return mid_auto(d);
}

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
