// Sustained-clock probe for bench.py (measurement infrastructure, not part of the attention C ABI):
// a pure v_mfma_f32_32x32x16_f16 loop on pseudo-random f16 operands, one 256-thread workgroup per
// CU, 8 independent accumulator chains per wave. Each workgroup records the shader-clock cycles
// (s_memtime) its loop took; the caller times the launch with events, so cycles / time is the
// clock the MFMA units actually ran at under a full, data-dependent f16 load, and the launch's
// FLOP / time is the dense-f16 rate such a load reaches. Built into libmiso_probe.so.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));

__global__ void __launch_bounds__(256) mfma_clock_kernel(float* out, long long* cycles,
                                                         unsigned iters) {
  half8_t a[16], b[16];
  unsigned h = threadIdx.x * 2654435761u + blockIdx.x * 40503u + 12345u;
  for (int j = 0; j < 16; ++j)
    for (int i = 0; i < 8; ++i) {  // uniform in [-1, 1), different per lane and register
      h = h * 1664525u + 1013904223u;
      a[j][i] = static_cast<_Float16>(((h >> 8) & 0xffffu) / 32768.0f - 1.0f);
      h = h * 1664525u + 1013904223u;
      b[j][i] = static_cast<_Float16>(((h >> 8) & 0xffffu) / 32768.0f - 1.0f);
    }
  float16_t acc[8];
  for (int c = 0; c < 8; ++c)
    acc[c] = float16_t{};
  __syncthreads();
  const long long t0 = __builtin_readcyclecounter();
  for (unsigned it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      acc[j % 8] =
          __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j], b[(j * 5) % 16], acc[j % 8], 0, 0, 0);
  }
  const long long t1 = __builtin_readcyclecounter();
  float s = 0.0f;
  for (int c = 0; c < 8; ++c)
    for (int r = 0; r < 16; ++r)
      s += acc[c][r];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if (threadIdx.x == 0)
    cycles[blockIdx.x] = t1 - t0;
}

}  // namespace

// out: blocks * 256 floats; cycles: blocks entries. 16 * iters MFMAs per wave, 4 waves per block.
extern "C" int miso_probe_mfma_clock(float* out, long long* cycles, unsigned blocks,
                                     unsigned iters, void* stream) {
  if (out == nullptr || cycles == nullptr || blocks == 0 || iters == 0)
    return static_cast<int>(hipErrorInvalidValue);
  hipLaunchKernelGGL(mfma_clock_kernel, dim3(blocks), dim3(256), 0,
                     static_cast<hipStream_t>(stream), out, cycles, iters);
  return static_cast<int>(hipGetLastError());
}
