#pragma once

// Q6_K GEMV y = W x for MI355X (gfx950 / CDNA4), f16 activations: the attention's attn_v
// projection (2048 -> 512, Q6_K in the engine's model). Same names, fields and template
// parameters as miso's kernels/q6k_gemv.hpp (Q6kGemvParams, q6k_gemv_op<K, kBlock, kRows>,
// q6k_gemv_kernel<K, kBlock, kRows>); the body is new.
//
// Weights are Q6_K "r1" rows (src/repack.hpp:25-28): a row of nb = K / 256 GGUF blocks stored as
// [ql: nb x 128][qh: nb x 64][scales: nb x 16 int8][d: nb x 2 f16], zero-padded to 16 bytes.
// Element e of block b: q6 = ql nibble | qh 2-bit pair << 4 (ql[b][64 (e / 128) + e % 64] >>
// 4 (e % 128 / 64), qh[b][32 (e / 128) + e % 32] >> 2 (e % 128 / 32)), w = d sc[e / 16] (q6 - 32).
//
// Mapping: 8 lanes per block; lane j of a block takes half h = j / 4 and columns
// c = 16 (j % 4) .. c + 15 of it: its 16 ql bytes hold elements 128h + c + t (low nibbles) and
// 128h + 64 + c + t (high nibbles), t < 16, and the 16 qh bytes at 32h + c % 32 hold both sets'
// top bits. Codes enter v_dot2_f32_f16 as f16 subnormal pairs (q6 2^-24, exact); the - 32
// offset is applied once per 16 elements through the sum of the converted activations.

#include "q4k_gemv.hpp"

namespace miso::kernels {

struct Q6kGemvParams {
  const std::uint8_t* w;  // n_rows Q6_K r1 rows of K / 256 blocks
  const float* x;         // K activations
  float* y;               // n_rows outputs
  unsigned n_rows;
};

namespace q6k_gemv_detail {

using q4k_gemv_detail::half2_t;
using q4k_gemv_detail::u32x4;
constexpr int kLanes = 64;

// 16 activations as f16 pairs in the order the masks below produce codes: ev[i] = (x[4i],
// x[4i + 2]), od[i] = (x[4i + 1], x[4i + 3]); sum of the converted values.
struct Half16 {
  half2_t ev[4], od[4];
  float sum;
};

__device__ inline Half16 half16(const float* x) {
  float v[16];
  q4k_gemv_detail::load16f(x, v);
  Half16 r;
  r.sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r.ev[i] = q4k_gemv_detail::pair(v[4 * i], v[4 * i + 2]);
    r.od[i] = q4k_gemv_detail::pair(v[4 * i + 1], v[4 * i + 3]);
    r.sum += (static_cast<float>(r.ev[i][0]) + static_cast<float>(r.ev[i][1])) +
             (static_cast<float>(r.od[i][0]) + static_cast<float>(r.od[i][1]));
  }
  return r;
}

// The lane's activations for one chunk (block c / 8, lane j = c % 8 of it): the low set
// 128h + 16 (j % 4) + t and the high set 64 elements further.
struct ChunkX {
  Half16 lo, hi;
};

__device__ inline ChunkX convert_chunk(const float* x, unsigned c) {
  const unsigned j = c & 7u;
  const float* p = x + 256 * (c >> 3) + 128 * (j >> 2) + 16 * (j & 3u);
  return {half16(p), half16(p + 64)};
}

struct ChunkW {
  u32x4 ql, qh;
  unsigned sc;      // the two int8 scales of the low and high sets, in bytes 0 and 1
  unsigned d_bits;  // f16 d in the low 16 bits
};

template <unsigned K>
__device__ __attribute__((always_inline)) inline ChunkW load_chunk(const std::uint8_t* row,
                                                                   unsigned c) {
  constexpr unsigned nb = K / 256;
  const unsigned b = c >> 3, j = c & 7u, h = j >> 2, col = 16 * (j & 3u);
  ChunkW w;
  w.ql = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + 128 * b + 64 * h + col));
  w.qh = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(row + nb * 128 + 64 * b + 32 * h + (col & 31u)));
  const std::uint8_t* sc = row + nb * 192 + 16 * b + 8 * h + (j & 3u);
  w.sc = static_cast<unsigned>(sc[0]) | static_cast<unsigned>(sc[4]) << 8;
  w.d_bits = *reinterpret_cast<const unsigned short*>(row + nb * 208 + 2 * b);
  return w;
}

// Codes of bytes 0 and 2 (s = 0 / 4 for the low / high nibble, u = the qh shift) or of bytes 1
// and 3 (s + 8, u + 8) as an f16 subnormal pair.
__device__ __attribute__((always_inline)) inline half2_t code_pair(unsigned ql, unsigned s,
                                                                   unsigned qh, unsigned u) {
  return __builtin_bit_cast(half2_t,
                            ((ql >> s) & 0x000F000Fu) | (((qh >> u) & 0x00030003u) << 4));
}

__device__ __attribute__((always_inline)) inline float chunk_dot(const ChunkW& w, unsigned c,
                                                                 const ChunkX& x) {
  const unsigned col = 16 * (c & 3u);
  const unsigned u_lo = 2 * (col >> 5), u_hi = u_lo + 4;
  const unsigned ql[4] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w};
  const unsigned qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo = __builtin_amdgcn_fdot2(code_pair(ql[i], 0, qh[i], u_lo), x.lo.ev[i], lo, false);
    lo = __builtin_amdgcn_fdot2(code_pair(ql[i], 8, qh[i], u_lo + 8), x.lo.od[i], lo, false);
    hi = __builtin_amdgcn_fdot2(code_pair(ql[i], 4, qh[i], u_hi), x.hi.ev[i], hi, false);
    hi = __builtin_amdgcn_fdot2(code_pair(ql[i], 12, qh[i], u_hi + 8), x.hi.od[i], hi, false);
  }
  const float sc_lo = static_cast<float>(static_cast<std::int8_t>(w.sc & 0xFFu));
  const float sc_hi = static_cast<float>(static_cast<std::int8_t>(w.sc >> 8));
  const float d = q4k_gemv_detail::half_bits(w.d_bits & 0xFFFFu);
  return d * (sc_lo * (0x1p24f * lo - 32.0f * x.lo.sum) +
              sc_hi * (0x1p24f * hi - 32.0f * x.hi.sum));
}

}  // namespace q6k_gemv_detail

// Rows [first, first + count) over logical_grid workgroups of kBlock threads; kRows consecutive
// rows per wave step, the first step's weights requested before the activations convert and
// each next step's before the current step's reductions.
template <unsigned K, int kBlock, int kRows = 1>
__device__ void q6k_gemv_op(const Q6kGemvParams& p, unsigned first, unsigned count,
                            unsigned logical_block = blockIdx.x,
                            unsigned logical_grid = gridDim.x) {
  using namespace q6k_gemv_detail;
  static_assert(K % (32 * kLanes) == 0, "K must be a multiple of 2048");
  static_assert(kBlock % kLanes == 0 && kRows >= 1, "whole waves, at least one row");
  constexpr unsigned kChunks = K / (32 * kLanes);
  constexpr std::size_t kRowBytes = (std::size_t{K} / 256 * 210 + 15) / 16 * 16;
  const unsigned lane = threadIdx.x % kLanes;
  const unsigned wave = logical_block * (kBlock / kLanes) + threadIdx.x / kLanes;
  const unsigned waves = logical_grid * (kBlock / kLanes);
  const unsigned end = first + count;
  auto load_rows = [&](unsigned r0, ChunkW (&w)[kRows][kChunks]) __attribute__((always_inline)) {
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const unsigned r = r0 + rr < end ? r0 + rr : end - 1;  // a tail row re-reads the last row
#pragma unroll
      for (unsigned i = 0; i < kChunks; ++i)
        w[rr][i] = load_chunk<K>(p.w + std::size_t{r} * kRowBytes, lane + kLanes * i);
    }
  };
  unsigned r0 = first + wave * kRows;
  ChunkW w[kRows][kChunks];
  if (r0 < end)
    load_rows(r0, w);
  ChunkX xs[kChunks];
#pragma unroll
  for (unsigned i = 0; i < kChunks; ++i)
    xs[i] = convert_chunk(p.x, lane + kLanes * i);
  for (; r0 < end; r0 += waves * kRows) {
    float acc[kRows];
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      acc[rr] = 0.0f;
#pragma unroll
      for (unsigned i = 0; i < kChunks; ++i)
        acc[rr] += chunk_dot(w[rr][i], lane + kLanes * i, xs[i]);
    }
    if (r0 + waves * kRows < end)
      load_rows(r0 + waves * kRows, w);
#pragma unroll
    for (int rr = 0; rr < kRows; ++rr) {
      const float sum = cdna4::wave_allsum(acc[rr]);
      if (lane == 0 && r0 + rr < end)
        p.y[r0 + rr] = sum;
    }
  }
}

template <unsigned K, int kBlock, int kRows = 1>
__global__ void __launch_bounds__(kBlock) q6k_gemv_kernel(Q6kGemvParams p) {
  q6k_gemv_op<K, kBlock, kRows>(p, 0, p.n_rows);
}

}  // namespace miso::kernels
