#pragma once

// Q4_K GEMV y = W x for MI355X (gfx950 / CDNA4): the decode-time projections on either side of
// the attention (attn_q 2048 -> 8192, attn_k 2048 -> 512, attn_output 4096 -> 2048 are Q4_K in the
// engine's model). Source-compatible with miso's kernels/q4k_gemv.hpp: ActFormat, Q4kGemvParams,
// q4k_gemv_op<A, K, kBlock, kRows>(params, first, count, logical_block, logical_grid) and
// q4k_gemv_kernel<A, K, kBlock, kRows> keep their names, fields and template parameters, so
// tests/test_q4k_gemv.hip compiles unchanged against it. (src/engine/weights.hip also includes the
// reference's kernels/qgemm.hpp, which includes the reference's q4k_gemv.hpp from its own
// directory; this header replaces that one only together with a qgemm.hpp, not provided here.)
// The body is new.
//
// Weights are Q4_K "r1" blocks (src/repack.hpp:14-19): the 144-byte GGUF block with bytes 4..15
// holding, per nibble group g (sub-blocks 2g, 2g + 1, whose nibbles share bytes 16 + 32g ..
// 16 + 32g + 31: low nibbles 2g, high nibbles 2g + 1), the 24-bit field
// sc[2g] | m[2g] << 6 | sc[2g+1] << 12 | m[2g+1] << 18 at byte 4 + 3g. w = d sc q - dmin m.
//
// Mapping: a row of K weights is K / 32 "chunks" of 16 nibble bytes (32 weights: 16 of a
// sub-block pair's low and 16 of its high sub-block). Lane l of a wave owns chunks l, l + 64, ...
// (K / 2048 of them) in every row; its activations are converted once per wave and kept in
// registers. A wave walks kRows rows per step with all their 16-byte loads (nibbles and block
// header, non-temporal: each weight is read once) issued before any arithmetic, then reduces each
// row across the wave with DPP.
//
// Arithmetic: Fp16 activations enter v_dot2_f32_f16 against nibble pairs placed in the f16
// subnormal range (q 2^-24, exact, no offset to cancel), so the f32 chain is exact up to its own
// rounding; Int8 activations (per-32 absmax / 127, round to nearest even) use v_dot4_i32_i8
// against the nibbles. The dmin m term uses the sum of the converted activations of each
// sub-block half, so it cancels against the q term's rounding of the same values.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "cdna4_wave.hpp"

namespace miso::kernels {

enum class ActFormat {
  Int8,  // per-32 absmax INT8 activations, v_dot4_i32_i8
  Fp16,  // FP16 activations, v_dot2_f32_f16
};

struct Q4kGemvParams {
  const std::uint8_t* w;  // n_rows rows of K / 256 Q4_K r1 blocks; rows 16-byte aligned
  const float* x;         // K activations
  float* y;               // n_rows outputs
  unsigned n_rows;
};

namespace q4k_gemv_detail {

using cdna4::half2_t;
constexpr unsigned kBlockBytes = 144;
constexpr int kLanes = 64;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// The lane's activations for one chunk: sub-block halves lo (2g) and hi (2g + 1), 16 values each,
// in the order the nibble extraction produces them, plus the sums of the converted values.
template <ActFormat A>
struct ChunkX;

template <>
struct ChunkX<ActFormat::Fp16> {
  // ev[c] = (x[4c], x[4c + 2]), od[c] = (x[4c + 1], x[4c + 3]) of the lo / hi half
  half2_t lo_ev[4], lo_od[4], hi_ev[4], hi_od[4];
  float sum_lo, sum_hi;
};

template <>
struct ChunkX<ActFormat::Int8> {
  unsigned lo[4], hi[4];  // 16 int8 each, natural order
  float step_lo, step_hi;  // activation = step * int8
  float sum_lo, sum_hi;    // step * sum of the int8 values
};

// 16 consecutive floats at p (16-byte aligned).
__device__ __attribute__((always_inline)) inline void load16f(const float* p, float (&v)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 f = reinterpret_cast<const float4*>(p)[i];
    v[4 * i] = f.x, v[4 * i + 1] = f.y, v[4 * i + 2] = f.z, v[4 * i + 3] = f.w;
  }
}

// Chunk c of a row: block c / 8, nibble bytes 16 (c % 8) .. + 15 of it, i.e. group g = c % 8 / 2,
// elements 16 (c % 2) .. + 15 of sub-blocks 2g (lo) and 2g + 1 (hi).
__device__ __attribute__((always_inline)) inline const float* chunk_x(const float* x, unsigned c) {
  return x + 256 * (c >> 3) + 64 * ((c >> 1) & 3u) + 16 * (c & 1u);
}

__device__ __attribute__((always_inline)) inline half2_t pair(float a, float b) {
  return half2_t{static_cast<_Float16>(a), static_cast<_Float16>(b)};
}

// Lane ^ 1's value (DPP quad permutation [1, 0, 3, 2]).
__device__ __attribute__((always_inline)) inline float swap_pair(float v) {
  return cdna4::as_float(__builtin_amdgcn_mov_dpp(cdna4::as_uint(v), 0xB1, 0xF, 0xF, false));
}

template <ActFormat A>
__device__ inline ChunkX<A> convert_chunk(const float* x, unsigned c) {
  float lo[16], hi[16];
  load16f(chunk_x(x, c), lo);
  load16f(chunk_x(x, c) + 32, hi);
  ChunkX<A> s;
  if constexpr (A == ActFormat::Fp16) {
    s.sum_lo = 0.0f;
    s.sum_hi = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s.lo_ev[i] = pair(lo[4 * i], lo[4 * i + 2]);
      s.lo_od[i] = pair(lo[4 * i + 1], lo[4 * i + 3]);
      s.hi_ev[i] = pair(hi[4 * i], hi[4 * i + 2]);
      s.hi_od[i] = pair(hi[4 * i + 1], hi[4 * i + 3]);
      s.sum_lo += (static_cast<float>(s.lo_ev[i][0]) + static_cast<float>(s.lo_ev[i][1])) +
                  (static_cast<float>(s.lo_od[i][0]) + static_cast<float>(s.lo_od[i][1]));
      s.sum_hi += (static_cast<float>(s.hi_ev[i][0]) + static_cast<float>(s.hi_ev[i][1])) +
                  (static_cast<float>(s.hi_od[i][0]) + static_cast<float>(s.hi_od[i][1]));
    }
  } else {
    // A sub-block's 32 activations are split between this lane and lane ^ 1 (chunks c, c ^ 1).
    float m_lo = 0.0f, m_hi = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      m_lo = fmaxf(m_lo, __builtin_fabsf(lo[i]));
      m_hi = fmaxf(m_hi, __builtin_fabsf(hi[i]));
    }
    m_lo = fmaxf(m_lo, swap_pair(m_lo));
    m_hi = fmaxf(m_hi, swap_pair(m_hi));
    s.step_lo = m_lo / 127.0f;
    s.step_hi = m_hi / 127.0f;
    const float inv_lo = m_lo > 0.0f ? 127.0f / m_lo : 0.0f;
    const float inv_hi = m_hi > 0.0f ? 127.0f / m_hi : 0.0f;
    int q_lo = 0, q_hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      unsigned pl = 0, ph = 0;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int a = static_cast<int>(__builtin_rintf(lo[4 * i + t] * inv_lo));
        const int b = static_cast<int>(__builtin_rintf(hi[4 * i + t] * inv_hi));
        pl |= (static_cast<unsigned>(a) & 0xFFu) << (8 * t);
        ph |= (static_cast<unsigned>(b) & 0xFFu) << (8 * t);
        q_lo += a;
        q_hi += b;
      }
      s.lo[i] = pl;
      s.hi[i] = ph;
    }
    s.sum_lo = s.step_lo * static_cast<float>(q_lo);
    s.sum_hi = s.step_hi * static_cast<float>(q_hi);
  }
  return s;
}

// One chunk of one row: its block header and its 16 nibble bytes.
struct ChunkW {
  u32x4 head, nib;
};

__device__ __attribute__((always_inline)) inline ChunkW load_chunk(const std::uint8_t* row,
                                                                   unsigned c) {
  const std::uint8_t* blk = row + kBlockBytes * (c >> 3);
  return {__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(blk)),
          __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(blk + 16 + 16 * (c & 7u)))};
}

__device__ __attribute__((always_inline)) inline float half_bits(unsigned h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// The 24-bit (sc0, m0, sc1, m1) field of nibble group g: bytes 4 + 3g .. 6 + 3g of the header,
// i.e. bits 24g .. 24g + 23 of header words 1..3 taken as one 96-bit little-endian value.
__device__ __attribute__((always_inline)) inline unsigned group_field(const u32x4& h, unsigned g) {
  const unsigned lo = g == 0 ? h.y : g == 1 ? h.y : g == 2 ? h.z : h.w;
  const unsigned hi = g == 0 ? h.z : g == 1 ? h.z : g == 2 ? h.w : h.w;
  const unsigned shift = g == 0 ? 0u : g == 1 ? 24u : g == 2 ? 16u : 8u;
  return __builtin_amdgcn_alignbit(hi, lo, shift) & 0xFFFFFFu;
}

// Nibbles at bits s and s + 16 of w as an f16 pair in the subnormal range: (q, q') 2^-24.
__device__ __attribute__((always_inline)) inline half2_t nib_pair(unsigned w, unsigned s) {
  return __builtin_bit_cast(half2_t, (w >> s) & 0x000F000Fu);
}

template <ActFormat A>
__device__ __attribute__((always_inline)) inline float chunk_dot(const ChunkW& w, unsigned c,
                                                                 const ChunkX<A>& x) {
  const unsigned f = group_field(w.head, (c >> 1) & 3u);
  const float sc0 = static_cast<float>(f & 63u), m0 = static_cast<float>((f >> 6) & 63u);
  const float sc1 = static_cast<float>((f >> 12) & 63u), m1 = static_cast<float>(f >> 18);
  const float d = half_bits(w.head.x & 0xFFFFu), dmin = half_bits(w.head.x >> 16);
  const unsigned q[4] = {w.nib.x, w.nib.y, w.nib.z, w.nib.w};
  const float mins = dmin * (m0 * x.sum_lo + m1 * x.sum_hi);
  if constexpr (A == ActFormat::Fp16) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo = __builtin_amdgcn_fdot2(nib_pair(q[i], 0), x.lo_ev[i], lo, false);
      lo = __builtin_amdgcn_fdot2(nib_pair(q[i], 8), x.lo_od[i], lo, false);
      hi = __builtin_amdgcn_fdot2(nib_pair(q[i], 4), x.hi_ev[i], hi, false);
      hi = __builtin_amdgcn_fdot2(nib_pair(q[i], 12), x.hi_od[i], hi, false);
    }
    return d * 0x1p24f * (sc0 * lo + sc1 * hi) - mins;
  } else {
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo = __builtin_amdgcn_sdot4(static_cast<int>(q[i] & 0x0F0F0F0Fu), static_cast<int>(x.lo[i]),
                                  lo, false);
      hi = __builtin_amdgcn_sdot4(static_cast<int>((q[i] >> 4) & 0x0F0F0F0Fu),
                                  static_cast<int>(x.hi[i]), hi, false);
    }
    return d * (sc0 * x.step_lo * static_cast<float>(lo) +
                sc1 * x.step_hi * static_cast<float>(hi)) - mins;
  }
}

}  // namespace q4k_gemv_detail

// Rows [first, first + count) over logical_grid workgroups of kBlock threads (the reference's
// fused callers pass their own block index and grid). Each wave takes kRows consecutive rows per
// step and strides by the number of waves; its first rows' weights are requested before the
// activations are converted, and each next step's before the current step's reductions.
template <ActFormat A, unsigned K, int kBlock, int kRows = 1>
__device__ void q4k_gemv_op(const Q4kGemvParams& p, unsigned first, unsigned count,
                            unsigned logical_block = blockIdx.x,
                            unsigned logical_grid = gridDim.x) {
  using namespace q4k_gemv_detail;
  static_assert(K % (32 * kLanes) == 0, "K must be a multiple of 2048");
  static_assert(kBlock % kLanes == 0 && kRows >= 1, "whole waves, at least one row");
  constexpr unsigned kChunks = K / (32 * kLanes);  // chunks per lane and row
  constexpr std::size_t kRowBytes = std::size_t{K} / 256 * kBlockBytes;
  const unsigned lane = threadIdx.x % kLanes;
  const unsigned wave = logical_block * (kBlock / kLanes) + threadIdx.x / kLanes;
  const unsigned waves = logical_grid * (kBlock / kLanes);

  const unsigned end = first + count;
  // All 16-byte loads of the kRows rows at r0 (a tail row re-reads the last row).
  auto load_rows = [&](unsigned r0, ChunkW (&w)[kRows][kChunks]) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const unsigned r = r0 + rr < end ? r0 + rr : end - 1;
      const std::uint8_t* row = p.w + std::size_t{r} * kRowBytes;
#pragma unroll
      for (unsigned i = 0; i < kChunks; ++i)
        w[rr][i] = load_chunk(row, lane + kLanes * i);
    }
  };
  unsigned r0 = first + wave * kRows;
  ChunkW w[kRows][kChunks];
  if (r0 < end)
    load_rows(r0, w);  // the first rows' weights are in flight while the activations convert

  ChunkX<A> xs[kChunks];
#pragma unroll
  for (unsigned i = 0; i < kChunks; ++i)
    xs[i] = convert_chunk<A>(p.x, lane + kLanes * i);

  for (; r0 < end; r0 += waves * kRows) {
    float acc[kRows];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      acc[rr] = 0.0f;
#pragma unroll
      for (unsigned i = 0; i < kChunks; ++i)
        acc[rr] += chunk_dot<A>(w[rr][i], lane + kLanes * i, xs[i]);
    }
    if (r0 + waves * kRows < end)
      load_rows(r0 + waves * kRows, w);  // the next step's weights load under the reductions
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const float sum = cdna4::wave_allsum(acc[rr]);
      if (lane == 0 && r0 + rr < end)
        p.y[r0 + rr] = sum;
    }
  }
}

template <ActFormat A, unsigned K, int kBlock, int kRows = 1>
__global__ void __launch_bounds__(kBlock) q4k_gemv_kernel(Q4kGemvParams p) {
  q4k_gemv_op<A, K, kBlock, kRows>(p, 0, p.n_rows);
}

}  // namespace miso::kernels
