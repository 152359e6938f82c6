// LDS read probe for bench.py (measurement infrastructure, not part of the attention C ABI): the
// operand reads one 32-key tile costs the causal prefill, without the MFMAs. One workgroup of 4
// waves per CU (the prefill's shape); every wave reads a K tile and a V tile of the prefill's LDS
// layout (prefill_detail::swz_k / swz_v) with the prefill's instructions and addresses:
//   K: 16 ds_read_b128 at (col 512 + 16 (hi ^ (col % 16))) ^ 32 st          (16 KiB per wave)
//   V: 32 ds_read_b64_tr_b16 at the transpose-read bases of the four 32-dim blocks (16 KiB)
// mode 0 = both (one tile), 1 = K only, 2 = V only. Each workgroup records the shader-clock
// cycles (s_memtime) per wave for `iters` tiles; cycles / iters is the LDS time of one tile per
// CU, since the four waves share the CU's LDS. Built into libmiso_probe.so.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attention_prefill.hpp"

namespace {

using miso::kernels::prefill_detail::kRowBytes;
using miso::kernels::prefill_detail::kTileBytes;
using miso::kernels::prefill_detail::swz_v;
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef __fp16 lds_fp16x4 __attribute__((vector_size(8)));

template <int kMode>
__global__ void __launch_bounds__(256) lds_tile_kernel(float* out, long long* cycles,
                                                       unsigned iters) {
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * kTileBytes];
  const unsigned t = threadIdx.x, lane = t & 63u, col = lane & 31u, hi = lane >> 5;
  for (unsigned i = t; i < 2 * kTileBytes / 4; i += 256)
    reinterpret_cast<unsigned*>(lds)[i] = i * 2654435761u;
  __syncthreads();
  const unsigned l0 = miso::kernels::cdna4::lds_offset(lds);
  const unsigned kb = l0 + col * kRowBytes + 16 * (hi ^ (col & 15u));
  unsigned vb[4];
  {
    const unsigned g = lane >> 4, j = lane & 15u;
    const unsigned vrow = 4 * (g >> 1) + j / 4, vchunk = 2 * (g & 1u) + (j % 4) / 2;
    const unsigned base = vrow * kRowBytes + 8 * ((j % 4) & 1u) + 16 * swz_v(vrow, vchunk);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      vb[c] = l0 + kTileBytes + (base ^ (64u * c));
  }
  half8_t acc8 = {};
  half4_t acc4 = {};
  const long long t0 = __builtin_readcyclecounter();
  for (unsigned it = 0; it < iters; ++it) {
    asm volatile("" ::: "memory");  // every tile is read again
    if (kMode != 2) {
#pragma unroll
      for (unsigned st = 0; st < 16; ++st)
        acc8 += *reinterpret_cast<const __attribute__((address_space(3))) half8_t*>(kb ^ (32u * st));
    }
    if (kMode != 1) {
#pragma unroll
      for (unsigned i = 0; i < 16; ++i) {
        const unsigned b = i % 8, step = i / 8;
        const unsigned at = vb[b % 4] + 256u * (b / 4) + 8192u * step;
        const lds_fp16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) lds_fp16x4*>(at));
        const lds_fp16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
            reinterpret_cast<__attribute__((address_space(3))) lds_fp16x4*>(
                at + (b < 4 ? 4096u + 256u : 4096u - 256u)));
        acc4 += __builtin_bit_cast(half4_t, lo) + __builtin_bit_cast(half4_t, up);
      }
    }
  }
  const long long t1 = __builtin_readcyclecounter();
  float s = 0.0f;
  for (int i = 0; i < 8; ++i)
    s += static_cast<float>(acc8[i]);
  for (int i = 0; i < 4; ++i)
    s += static_cast<float>(acc4[i]);
  out[blockIdx.x * 256 + t] = s;
  if (lane == 0)
    cycles[blockIdx.x * 4 + (t >> 6)] = t1 - t0;
}

}  // namespace

// out: blocks * 256 floats; cycles: blocks * 4 entries (per wave).
extern "C" int miso_probe_lds_tile(float* out, long long* cycles, unsigned blocks, unsigned mode,
                                   unsigned iters, void* stream) {
  if (out == nullptr || cycles == nullptr || blocks == 0 || iters == 0 || mode > 2)
    return static_cast<int>(hipErrorInvalidValue);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (mode == 0)
    hipLaunchKernelGGL(lds_tile_kernel<0>, dim3(blocks), dim3(256), 0, s, out, cycles, iters);
  else if (mode == 1)
    hipLaunchKernelGGL(lds_tile_kernel<1>, dim3(blocks), dim3(256), 0, s, out, cycles, iters);
  else
    hipLaunchKernelGGL(lds_tile_kernel<2>, dim3(blocks), dim3(256), 0, s, out, cycles, iters);
  return static_cast<int>(hipGetLastError());
}
