// Measurement helper, not part of the t0hip C ABI: a plain streaming read of a
// device buffer, the reference point the benchmark prices the bandwidth-bound
// GEMV launches against (the time one launch needs to read the same bytes once,
// timed the same way).  Each thread reads sixteen 16-byte chunks, 4096 chunks
// (64 KiB) a workgroup, coalesced across the wave; the loaded words are folded
// with XOR and one word a workgroup is stored, so no load is optimised away.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int SR_U = 16;

__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ p, size_t n16, uint32_t* out) {
  const size_t base = (size_t)blockIdx.x * 256 * SR_U + threadIdx.x;
  uint4 v[SR_U];
#pragma unroll
  for (int u = 0; u < SR_U; ++u) {
    const size_t i = base + (size_t)u * 256;
    v[u] = p[i < n16 ? i : n16 - 1];
  }
  uint32_t a = 0;
#pragma unroll
  for (int u = 0; u < SR_U; ++u) a ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  __shared__ uint32_t s[256];
  s[threadIdx.x] = a;
  __syncthreads();
  if (threadIdx.x < 64) {
    uint32_t t = s[threadIdx.x] ^ s[threadIdx.x + 64] ^ s[threadIdx.x + 128] ^ s[threadIdx.x + 192];
    for (int o = 32; o > 0; o >>= 1) t ^= __shfl_xor(t, o);
    if (threadIdx.x == 0) out[blockIdx.x] = t;
  }
}

}  // namespace

// Reads bytes (a multiple of 16, at least 16) at p once; out receives one word per
// 64 KiB (t0p_stream_read_out_words of them).  0 on success, else a hipError_t.
extern "C" size_t t0p_stream_read_out_words(size_t bytes) { return (bytes / 16 + 256 * SR_U - 1) / (256 * SR_U); }

extern "C" int t0p_stream_read(const void* p, size_t bytes, void* out, void* stream) {
  if (!p || !out || bytes < 16 || bytes % 16) return (int)hipErrorInvalidValue;
  const size_t n16 = bytes / 16;
  hipLaunchKernelGGL(k_stream_read, dim3((unsigned)t0p_stream_read_out_words(bytes)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const uint4*>(p), n16, static_cast<uint32_t*>(out));
  return (int)hipGetLastError();
}
