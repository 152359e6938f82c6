#pragma once

// CDNA4 (gfx950) wavefront primitives for the attention kernels. They live in the nested
// namespace miso::kernels::cdna4 and in a file of their own name, so a translation unit that also
// includes another kernels header with its own miso::kernels wave helpers (kWave, dpp, wave_sum,
// block_sum, ...) sees no duplicate definitions.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace miso::kernels::cdna4 {

constexpr int kLanes = 64;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

__device__ inline unsigned lane_id() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

__device__ inline float as_float(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ inline unsigned as_uint(float f) { return __builtin_bit_cast(unsigned, f); }
__device__ inline half2_t as_half2(unsigned u) { return __builtin_bit_cast(half2_t, u); }
__device__ inline unsigned as_uint(half2_t h) { return __builtin_bit_cast(unsigned, h); }

// DPP controls used here (gfx9 encoding).
constexpr int kQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kRowRor8 = 0x128;        // row_ror:8 inside a 16-lane row: lane ^ 8
constexpr int kRowMirror = 0x140;      // lane i of a 16-lane row <- lane 15 - i
constexpr int kRowHalfMirror = 0x141;  // lane i of an 8-lane half-row <- lane 7 - i

// DPP move of v with every row and bank enabled (all controls above have a source in range).
template <int kCtrl>
__device__ inline float dpp_mov(float v) {
  return as_float(__builtin_amdgcn_update_dpp(0u, as_uint(v), kCtrl, 0xF, 0xF, true));
}

// v_permlane16_swap / v_permlane32_swap (gfx950), as measured on MI355X:
//   swap16(x, y) -> {[x.r0, y.r0, x.r2, y.r2], [x.r1, y.r1, x.r3, y.r3]}   (r = 16-lane row)
//   swap32(x, y) -> {[x.lo, y.lo], [x.hi, y.hi]}                           (lo/hi = 32-lane half)
struct Pair {
  float a, b;
};
__device__ inline Pair swap16(float x, float y) {
  const auto r = __builtin_amdgcn_permlane16_swap(as_uint(x), as_uint(y), false, false);
  return {as_float(r[0]), as_float(r[1])};
}
__device__ inline Pair swap32(float x, float y) {
  const auto r = __builtin_amdgcn_permlane32_swap(as_uint(x), as_uint(y), false, false);
  return {as_float(r[0]), as_float(r[1])};
}

// op(v, value of lane ^ 16) and op(v, value of lane ^ 32), in every lane.
__device__ inline float sum_xor16(float v) {
  const Pair p = swap16(v, v);
  return p.a + p.b;
}
__device__ inline float max_xor16(float v) {
  const Pair p = swap16(v, v);
  return fmaxf(p.a, p.b);
}
__device__ inline float sum_xor32(float v) {
  const Pair p = swap32(v, v);
  return p.a + p.b;
}
__device__ inline float max_xor32(float v) {
  const Pair p = swap32(v, v);
  return fmaxf(p.a, p.b);
}

// Max / sum over all 64 lanes, returned in every lane.
__device__ inline float wave_allmax(float v) {
  v = fmaxf(v, dpp_mov<kQuadXor1>(v));
  v = fmaxf(v, dpp_mov<kQuadXor2>(v));
  v = fmaxf(v, dpp_mov<kRowHalfMirror>(v));
  v = fmaxf(v, dpp_mov<kRowMirror>(v));
  return max_xor32(max_xor16(v));
}

__device__ inline float wave_allsum(float v) {
  v += dpp_mov<kQuadXor1>(v);
  v += dpp_mov<kQuadXor2>(v);
  v += dpp_mov<kRowHalfMirror>(v);
  v += dpp_mov<kRowMirror>(v);
  return sum_xor32(sum_xor16(v));
}

// Value of lane ^ 32 (used where the op is not symmetric).
__device__ inline float lane_xor32(float v) {
  const Pair p = swap32(v, v);
  return lane_id() < 32 ? p.b : p.a;
}

// ------------------------------------------------------------------------------------------------
// Direct global -> LDS loads (gfx950 global_load_lds_dwordx4).
//
// One instruction moves 16 bytes per lane: lane i's global address -> LDS byte lds_base + 16 i
// (lds_base is wave-uniform and travels in M0; an instruction offset would shift both addresses,
// so none is used). The load is issued from inline assembly and waited for with an explicit
// vmcnt: the compiler then neither tracks it nor inserts its own conservative full wait before
// later LDS reads. An explicit vmcnt(n) is always safe as long as n counts only the LDS loads this
// wave issued after the one being waited for -- any other vector-memory op in between only makes
// the wait stricter, since vmcnt drains in issue order.
// ------------------------------------------------------------------------------------------------

__device__ inline unsigned lds_offset(const void* p) {
  return static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// M0 is saved and restored around the load, so code the compiler generated around it keeps
// whatever M0 held.
__device__ __attribute__((always_inline)) inline void lds_load16(const void* gaddr,
                                                                 unsigned lds_base) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(lds_base)
      : "memory");
}

// The same load with the non-temporal hint, for data streamed once (the KV cache in decode).
__device__ __attribute__((always_inline)) inline void lds_load16_nt(const void* gaddr,
                                                                    unsigned lds_base) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(lds_base)
      : "memory");
}

// Wait until at most N vector-memory ops of this wave are outstanding (LDS and VGPR loads both
// count); also a compiler barrier for memory.
template <int N>
__device__ __attribute__((always_inline)) inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// One reduce-scatter step over a pair of values (lo, hi). Lanes whose class bit is clear keep
// lo + partner's lo; lanes whose bit is set keep hi + partner's hi. The partner (given by
// `exchange`) always has the opposite class bit.
template <class Exchange>
__device__ inline float scatter_step(float lo, float hi, bool upper, Exchange exchange) {
  const float send = upper ? lo : hi;
  const float keep = upper ? hi : lo;
  return keep + exchange(send);
}

// Reduce-scatter of 32 per-lane partial values over the 32 lanes of each wave half.
// On entry lane c (= lane % 32) holds v[i], i = 0..31, partial sums over its own slice. On exit
// lane c returns sum over the 32 lanes c' of its half of v[c'][c]: the complete value with index
// c. Exchanges: lane ^ 16 (swap16), lane ^ 8, the 8-lane mirror (pairs i with 7 - i, so the opposite bit 2),
// lane ^ 2, lane ^ 1 -- every original lane is summed exactly once.
__device__ __attribute__((always_inline)) inline float reduce_scatter32(float (&v)[32]) {
  const unsigned c = lane_id() & 31u;
  float r16[16], r8[8], r4[4], r2[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {  // lane ^ 16: one swap16 moves both halves of the pair
    const Pair p = swap16(v[i], v[i + 16]);
    r16[i] = p.a + p.b;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
    r8[i] = scatter_step(r16[i], r16[i + 8], (c & 8u) != 0,
                         [](float x) { return dpp_mov<kRowRor8>(x); });
#pragma unroll
  for (int i = 0; i < 4; ++i)
    r4[i] = scatter_step(r8[i], r8[i + 4], (c & 4u) != 0,
                         [](float x) { return dpp_mov<kRowHalfMirror>(x); });
#pragma unroll
  for (int i = 0; i < 2; ++i)
    r2[i] = scatter_step(r4[i], r4[i + 2], (c & 2u) != 0,
                         [](float x) { return dpp_mov<kQuadXor2>(x); });
  return scatter_step(r2[0], r2[1], (c & 1u) != 0, [](float x) { return dpp_mov<kQuadXor1>(x); });
}

}  // namespace miso::kernels::cdna4
