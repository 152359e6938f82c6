#pragma once

// Prefill GEMM Y[t][n] = sum_k W[n][k] x[t][k] over Q4_K r1 / Q6_K r1 weights with f16 activations
// and f32 accumulation, for MI355X (gfx950 / CDNA4): the attention's q / k / v / output
// projections of a prefill chunk (src/engine/weights.hip:306-330 gemm_input / gemm, called from
// src/engine/attention.hip:125-146). The interface is miso's kernels/qgemm.hpp -- QFormat,
// QGemmActParams, qgemm_act_op / qgemm_act_kernel, QGemmParams, qgemm_op<F>, qgemm_tiles and
// qgemm_kernel<F> keep their names, fields and launch contract (qgemm_act_kernel on
// ceil(n_tok k / 32 / 256) workgroups of 256 threads, qgemm_kernel<F> on qgemm_tiles(n, n_tok)
// workgroups of 256 threads). The design is this file's own.
//
// Activations: qgemm_act rounds x to f16 (xh) and sums each 32-element group of the rounded
// values (xs, f32, in the reference's order), 8 elements per thread, the four threads of a quad
// combining a group's sum with DPP.
//
// GEMM: a workgroup computes a 64-token x 64-row tile with v_mfma_f32_32x32x16_f16, each of its 4
// waves a 32 x 32 quarter (the lane's accumulator column is one weight row, so per-row scales are
// per-lane scalars). K advances in stages of 128. Per stage every thread fetches (two stages
// ahead, into registers) 64 bytes of the x tile and one 16-byte run of one row's quantized
// weights, and expands the weights into LDS as exact f16 integers:
//   Q4_K: q sc (<= 945) per weight through the 1024-exponent convert and one fused v_pk_fma_f16;
//         a block's partial C (16 MFMAs over its 256 k) is scaled by the row's d, and the block's
//         dmin m term is one more MFMA: A = the tokens' 8 sub-block sums of the block, each split
//         into f16 hi and lo parts (xs 2^-6 = hi + lo 2^-11), against B = m and m 2^-11.
//   Q6_K: c - 32 (low nibble set) and 16 (c - 32) (high set), exact; each 16-element scale group
//         is one MFMA whose result the lane scales by d sc (d sc / 16 for the high set).
// LDS tiles are double-buffered by stage (one barrier per stage) and their 16-byte chunks are
// XOR-swizzled by row, so the 32 rows an MFMA operand read touches spread over the banks.
// Workgroups are mapped to tiles in groups of 8 token tiles swept across the row tiles, each XCD
// a contiguous part of that order, so an XCD's activations and weights are read from the memory
// side about once and reused through its L2.
//
// Q4_K products with at least 256 tiles of 128 x 128 can run qgemm_q4k_big_kernel instead (no
// reference counterpart; qgemm_big_tiles gives its grid, 0 where it does not pay): each wave a
// 64 x 64 quarter, so an LDS operand read feeds two MFMAs, with the dequantizing store of the
// next stage in the same step as the MFMAs; results bit-identical to qgemm_kernel's.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "cdna4_wave.hpp"
#include "q6k_gemv.hpp"

namespace miso::kernels {

enum class QFormat { Q4K, Q6K };

struct QGemmActParams {
  const float* x;  // n_tok x k
  _Float16* xh;    // n_tok x k, x rounded to FP16
  float* xs;       // n_tok x k / 32, sums of the rounded values of each 32-group
  unsigned k, n_tok;
};

struct QGemmParams {
  const std::uint8_t* w;  // n_rows rows in the format's r1 layout
  const _Float16* xh;     // n_tok x k
  const float* xs;        // n_tok x k / 32 (Q4_K only)
  float* y;               // n_tok rows of stride ldy
  unsigned k, n_rows, n_tok, ldy;
};

// Groups [first, first + count) of n_tok k / 32 (group g: elements 32 g .. 32 g + 31 of x, row
// major), grid-stride: thread i of the launch takes elements 8 (i % 4) .. + 7 of group
// first + i / 4. A group's sum is the reference's association (tests/test_qgemm.hip:92-104): the
// chunk sums ((h0 + h1) + h2) + h3 of its 8 four-element chunks added in order to 0, so xs is
// bit-identical to it; the quad's first lane gathers the other lanes' chunk sums by DPP broadcast.
__device__ inline void qgemm_act_op(const QGemmActParams& p, unsigned first, unsigned count) {
  const unsigned stride = gridDim.x * blockDim.x;  // a multiple of 4: quads stay whole
  for (unsigned i = blockIdx.x * blockDim.x + threadIdx.x; i / 4 < count; i += stride) {
    const std::size_t e = (std::size_t{first} + i / 4) * 32 + 8 * (i % 4);
    const float4 a = *reinterpret_cast<const float4*>(p.x + e);
    const float4 b = *reinterpret_cast<const float4*>(p.x + e + 4);
    const _Float16 h[8] = {static_cast<_Float16>(a.x), static_cast<_Float16>(a.y),
                           static_cast<_Float16>(a.z), static_cast<_Float16>(a.w),
                           static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
                           static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v[j] = static_cast<float>(h[j]);
    const float c0 = ((v[0] + v[1]) + v[2]) + v[3];
    const float c1 = ((v[4] + v[5]) + v[6]) + v[7];
    // Chunk sums 2 l and 2 l + 1 come from quad lane l (DPP quad_perm broadcasts of lane l).
    using cdna4::as_float;
    using cdna4::as_uint;
    auto from = [](float x, auto ctrl) {
      return as_float(__builtin_amdgcn_update_dpp(0u, as_uint(x), decltype(ctrl)::value, 0xF, 0xF,
                                                  true));
    };
    using L0 = std::integral_constant<int, 0x00>;
    using L1 = std::integral_constant<int, 0x55>;
    using L2 = std::integral_constant<int, 0xAA>;
    using L3 = std::integral_constant<int, 0xFF>;
    float sum = 0.0f + from(c0, L0{});
    sum += from(c1, L0{});
    sum += from(c0, L1{});
    sum += from(c1, L1{});
    sum += from(c0, L2{});
    sum += from(c1, L2{});
    sum += from(c0, L3{});
    sum += from(c1, L3{});
    *reinterpret_cast<uint4*>(p.xh + e) = __builtin_bit_cast(uint4, h);
    if (i % 4 == 0)
      p.xs[first + i / 4] = sum;
  }
}

// A template with a defaulted parameter: launches keep the reference's qgemm_act_kernel<<<...>>>
// form, and several translation units may include this header without clashing symbols.
template <int = 0>
__global__ void __launch_bounds__(256) qgemm_act_kernel(QGemmActParams p) {
  qgemm_act_op(p, 0, p.n_tok * (p.k / 32));
}

namespace qgemm_detail {

using cdna4::float16_t;
using cdna4::half2_t;
using cdna4::half8_t;
using q4k_gemv_detail::u32x4;

constexpr int kThreads = 256;
constexpr unsigned kBM = 64, kBN = 64, kBK = 128;  // tokens, rows, k per stage
constexpr unsigned kChunks = kBK / 8;              // 16-byte chunks per tile row

template <QFormat F>
constexpr unsigned row_bytes(unsigned k) {
  return F == QFormat::Q4K ? k / 256 * 144 : (k / 256 * 210 + 15) / 16 * 16;
}

// Half offset of chunk c of row r in a [rows][kBK] f16 tile (swizzled).
__device__ __attribute__((always_inline)) inline unsigned chunk_at(unsigned r, unsigned c) {
  return 8u * (kChunks * r + (c ^ (r & (kChunks - 1))));
}

struct alignas(16) Lds {
  _Float16 x[2][kBM * kBK];  // activations of the stage, by stage parity
  _Float16 w[2][kBN * kBK];  // expanded weights of the stage
  _Float16 xm[2][kBM][16];   // Q4_K, by block parity: sub-block sums as (hi, lo) pairs
  _Float16 wm[2][kBN][16];   // Q4_K: (m, m 2^-11) per sub-block
  float dd[2][kBN][4];       // Q4_K: d, dmin 2^6 (two unused slots: every quad lane writes one)
  float sc[2][kBN][8];       // Q6_K, by stage parity: d sc of the stage's 8 scale groups
};

// One thread's global data for a stage: x chunks 4q .. 4q + 3 of token tok, and 16 bytes of row
// tok's (as a weight row) quantized weights. q = thread % 4, tok = thread / 4. The loads have no
// control flow around them (a token or row past the end reads the last one, a stage past the end
// the last stage; store() zeroes what is out of range), so nothing waits for them before store()
// consumes them two stages later.
template <QFormat F>
struct Fetch;

template <>
struct Fetch<QFormat::Q4K> {
  u32x4 x[4];
  u32x4 head;  // block header
  u32x4 nib;   // nibble bytes 16 (q % 2) .. of group 2 (s % 2) + q / 2
  float2 xs;   // sums of sub-blocks 2q, 2q + 1 of the stage's block for token tok
};

template <>
struct Fetch<QFormat::Q6K> {
  u32x4 x[4];
  u32x4 ql;         // ql bytes 16 q .. 16 q + 15 of the stage's half-block
  u32x4 qh;         // qh bytes 16 (q % 2) ..
  unsigned short sc_lo, sc_hi;  // scale bytes 2 (q / 2), + 1 and 4 + 2 (q / 2), + 1 of the stage
  unsigned short d_bits;        // f16 d
};

template <QFormat F>
__device__ inline Fetch<F> fetch(const QGemmParams& p, unsigned n0, unsigned m0, unsigned s,
                                 unsigned t) {
  Fetch<F> f;
  const unsigned tok = t >> 2, q = t & 3u;
  const unsigned n_stages = p.k / kBK;
  s = s < n_stages ? s : n_stages - 1;
  const unsigned tk = m0 + tok < p.n_tok ? m0 + tok : p.n_tok - 1;
  const _Float16* xr = p.xh + std::size_t{tk} * p.k + kBK * s + 32 * q;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f.x[i] = *reinterpret_cast<const u32x4*>(xr + 8 * i);
  const unsigned row = n0 + tok < p.n_rows ? n0 + tok : p.n_rows - 1;
  const std::uint8_t* wr = p.w + std::size_t{row} * row_bytes<F>(p.k);
  const unsigned b = s / 2, part = s % 2;
  if constexpr (F == QFormat::Q4K) {
    const std::uint8_t* blk = wr + 144 * b;
    f.head = *reinterpret_cast<const u32x4*>(blk);
    f.nib = *reinterpret_cast<const u32x4*>(blk + 16 + 64 * part + 16 * q);
    f.xs = *reinterpret_cast<const float2*>(p.xs + std::size_t{tk} * (p.k / 32) + 8 * b + 2 * q);
  } else {
    const unsigned nb = p.k / 256;
    f.ql = *reinterpret_cast<const u32x4*>(wr + 128 * b + 64 * part + 16 * q);
    f.qh = *reinterpret_cast<const u32x4*>(wr + nb * 128 + 64 * b + 32 * part + 16 * (q & 1u));
    const std::uint8_t* sc = wr + nb * 192 + 16 * b + 8 * part + 2 * (q / 2);
    f.sc_lo = *reinterpret_cast<const unsigned short*>(sc);
    f.sc_hi = *reinterpret_cast<const unsigned short*>(sc + 4);
    f.d_bits = *reinterpret_cast<const unsigned short*>(wr + nb * 208 + 2 * b);
  }
  return f;
}

__device__ __attribute__((always_inline)) inline void put(_Float16* tile, unsigned r, unsigned c,
                                                          u32x4 v) {
  *reinterpret_cast<u32x4*>(tile + chunk_at(r, c)) = v;
}

// (hi, lo) with v 2^-6 = hi + lo 2^-11 up to f16 rounding of lo; |v| < 2^21 keeps hi finite.
__device__ __attribute__((always_inline)) inline half2_t split(float v) {
  const float s = v * 0x1p-6f;
  const _Float16 hi = static_cast<_Float16>(s);
  return half2_t{hi, static_cast<_Float16>((s - static_cast<float>(hi)) * 0x1p11f)};
}

// Writes a fetched stage into the stage-parity buffers (and, for Q4_K, its block's min-term
// operands and scales into the block-parity ones; both stages of a block write the same values,
// which are read only after the block's second barrier). The thread's token and row go to tile
// row off + t / 4.
template <QFormat F, class L = Lds>
__device__ inline void store(const Fetch<F>& f, L& sm, unsigned s, unsigned t, bool tok_ok,
                             bool row_ok, unsigned off = 0) {
  using q4k_gemv_detail::spread_bytes;
  const unsigned tok = off + (t >> 2), q = t & 3u, buf = s & 1u;
  const u32x4 zero{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    put(sm.x[buf], tok, 4 * q + i, tok_ok ? f.x[i] : zero);
  if constexpr (F == QFormat::Q4K) {
    using q4k_gemv_detail::int_pair;
    using q4k_gemv_detail::splat;
    const unsigned w[4] = {f.nib.x, f.nib.y, f.nib.z, f.nib.w};
    const unsigned j = 2 * (s % 2) + q / 2, hb = q & 1u;
    const u32x4 head = row_ok ? f.head : zero;  // a row past the end: all scales zero
    const unsigned fld = q4k_gemv_detail::scale_field(head, j);
    const float sc_lo = static_cast<float>(fld & 63u), sc_hi = static_cast<float>((fld >> 12) & 63u);
    const half2_t s_lo = splat(sc_lo), c_lo = splat(-1024.0f * sc_lo);
    const half2_t s_hi = splat(sc_hi * 0.0625f), c_hi = splat(-64.0f * sc_hi);
    unsigned lo[8], hi[8];
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const unsigned b = spread_bytes(w[d], i);
        lo[2 * d + i] = cdna4::as_uint(int_pair(b, 0x000F000Fu, s_lo, c_lo));
        hi[2 * d + i] = cdna4::as_uint(int_pair(b, 0x00F000F0u, s_hi, c_hi));
      }
    // Local k of the low set: 64 (q / 2) + 16 hb + i; of the high set 32 more.
    const unsigned c0 = 8 * (q / 2) + 2 * hb;
    put(sm.w[buf], tok, c0, u32x4{lo[0], lo[1], lo[2], lo[3]});
    put(sm.w[buf], tok, c0 + 1, u32x4{lo[4], lo[5], lo[6], lo[7]});
    put(sm.w[buf], tok, c0 + 4, u32x4{hi[0], hi[1], hi[2], hi[3]});
    put(sm.w[buf], tok, c0 + 5, u32x4{hi[4], hi[5], hi[6], hi[7]});
    {  // both stages of a block write the same block data (read after the block's second barrier)
      const unsigned bb = (s / 2) & 1u;
      const unsigned g = q4k_gemv_detail::scale_field(head, q);  // sub-blocks 2q, 2q + 1
      const float m0 = static_cast<float>((g >> 6) & 63u), m1 = static_cast<float>(g >> 18);
      const half2_t wm0{static_cast<_Float16>(m0), static_cast<_Float16>(m0 * 0x1p-11f)};
      const half2_t wm1{static_cast<_Float16>(m1), static_cast<_Float16>(m1 * 0x1p-11f)};
      *reinterpret_cast<uint2*>(&sm.wm[bb][tok][4 * q]) =
          uint2{cdna4::as_uint(wm0), cdna4::as_uint(wm1)};
      const float2 xs = tok_ok ? f.xs : float2{0.0f, 0.0f};
      *reinterpret_cast<uint2*>(&sm.xm[bb][tok][4 * q]) =
          uint2{cdna4::as_uint(split(xs.x)), cdna4::as_uint(split(xs.y))};
      const float dq = q == 0 ? q4k_gemv_detail::f16_bits(head.x & 0xFFFFu)
                              : q4k_gemv_detail::f16_bits(head.x >> 16) * 0x1p6f;
      sm.dd[bb][tok][q] = dq;  // slot 0: d, 1: dmin 2^6 (slots 2, 3 unused)
    }
  } else {
    using q6k_gemv_detail::code_pairs;
    const unsigned l[4] = {f.ql.x, f.ql.y, f.ql.z, f.ql.w};
    const unsigned h[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
    unsigned lo[8], hi[8];
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const q6k_gemv_detail::CodePairs c = code_pairs(l[d], h[d], i, 2 * (q / 2));
        lo[2 * d + i] = cdna4::as_uint(c.lo);
        hi[2 * d + i] = cdna4::as_uint(c.hi16);
      }
    // Elements 16 q + i (low set) and 64 + 16 q + i (high set) of the half-block.
    put(sm.w[buf], tok, 2 * q, u32x4{lo[0], lo[1], lo[2], lo[3]});
    put(sm.w[buf], tok, 2 * q + 1, u32x4{lo[4], lo[5], lo[6], lo[7]});
    put(sm.w[buf], tok, 8 + 2 * q, u32x4{hi[0], hi[1], hi[2], hi[3]});
    put(sm.w[buf], tok, 9 + 2 * q, u32x4{hi[4], hi[5], hi[6], hi[7]});
    const float d = row_ok ? q4k_gemv_detail::f16_bits(f.d_bits) : 0.0f;
    const unsigned at = 8 * (q & 1u);  // scale bytes q and 4 + q of the stage
    sm.sc[buf][tok][q] = d * static_cast<float>(static_cast<signed char>((f.sc_lo >> at) & 0xFFu));
    sm.sc[buf][tok][4 + q] =
        d * 0.0625f * static_cast<float>(static_cast<signed char>((f.sc_hi >> at) & 0xFFu));
  }
}

__device__ __attribute__((always_inline)) inline float16_t mfma(half8_t a, half8_t b,
                                                                float16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Tile index for workgroup b of a launch of `count` workgroups: workgroups are dealt round-robin
// to the 8 XCDs, so XCD x's workgroups b = x, x + 8, ... take the contiguous range
// [x q + min(x, r), ...) (q = count / 8, r = count % 8) of the tile order below.
__device__ __attribute__((always_inline)) inline unsigned xcd_tile(unsigned b, unsigned count) {
  const unsigned q = count / 8, r = count % 8, x = b % 8;
  return x * q + (x < r ? x : r) + b / 8;
}

// The tile order: groups of kGroupTok token tiles, and inside a group the row tiles in order, the
// group's token tiles fastest. The ~64 workgroups an XCD runs at once then cover 8 token tiles x 8
// row tiles, and a group's activations (8 x 64 tokens x k f16: 2 MiB at k = 2048) stay in that
// XCD's L2 while its row tiles pass -- each XCD reads its activations once and each weight row
// once per group, where a row tile swept across all token tiles would re-read the whole activation
// matrix from the memory side for every row tile.
constexpr unsigned kGroupTok = 8;
template <unsigned kGroup = kGroupTok>
__device__ __attribute__((always_inline)) inline void grouped_tile(unsigned t, unsigned n_ttiles,
                                                                  unsigned n_rtiles,
                                                                  unsigned& ttile,
                                                                  unsigned& rtile) {
  const unsigned per_group = kGroup * n_rtiles;
  const unsigned first_tok = t / per_group * kGroup, in = t % per_group;
  const unsigned width = n_ttiles - first_tok < kGroup ? n_ttiles - first_tok : kGroup;
  ttile = first_tok + in % width;
  rtile = in / width;
}

}  // namespace qgemm_detail

namespace qgemm_detail {

// One 64 x 64 output tile at tokens m0, rows n0. kStages: the stage count k / kBK when it is a
// compile-time constant (then the stage loop unrolls and the compiler's wait counts see the
// two-stage prefetch in straight-line code), 0 for any other k.
template <QFormat F, unsigned kStages>
__device__ __attribute__((always_inline)) inline void gemm_tile(const QGemmParams& p, Lds& sm,
                                                                unsigned m0, unsigned n0) {
  const unsigned t = threadIdx.x, lane = t % 64, wave = t / 64;
  const unsigned wt = wave >> 1, wr = wave & 1u;  // the wave's token half and row half
  const unsigned ar = 32 * wt + lane % 32, br = 32 * wr + lane % 32, kq = lane / 32;
  const unsigned n_stages = kStages ? kStages : p.k / kBK;
  float16_t acc = {}, c = {};
  // Two register sets, even and odd stages: stage s's data is requested two stages ahead.
  Fetch<F> fa = fetch<F>(p, n0, m0, 0, t);
  asm volatile("" : : : "memory");  // stage 0's loads are issued before stage 1's
  Fetch<F> fb = fetch<F>(p, n0, m0, 1, t);
  const bool tok_ok = m0 + t / 4 < p.n_tok, row_ok = n0 + t / 4 < p.n_rows;
  auto step = [&](Fetch<F>& f, unsigned s) __attribute__((always_inline)) {
    // Nothing crosses a stage boundary: the scheduler would otherwise hoist arithmetic on the
    // newest loads into the stage before, and the wait for them with it.
    __builtin_amdgcn_sched_barrier(0);
    store<F>(f, sm, s, t, tok_ok, row_ok);
    f = fetch<F>(p, n0, m0, s + 2, t);  // past the last stage: re-reads it, never stored
    __syncthreads();
    const unsigned buf = s & 1u;
#pragma unroll
    for (unsigned kk = 0; kk < kBK / 16; ++kk) {
      const half8_t a = *reinterpret_cast<const half8_t*>(sm.x[buf] + chunk_at(ar, 2 * kk + kq));
      const half8_t b = *reinterpret_cast<const half8_t*>(sm.w[buf] + chunk_at(br, 2 * kk + kq));
      if constexpr (F == QFormat::Q4K) {
        c = mfma(a, b, c);
      } else {
        const float16_t g = mfma(a, b, float16_t{});
        const float scale = sm.sc[buf][br][kk];
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[r] = __builtin_fmaf(scale, g[r], acc[r]);
      }
    }
    if constexpr (F == QFormat::Q4K) {
      if (s % 2 == 1) {  // the block's last stage: its dmin m term, then its d scale
        const unsigned bb = (s / 2) & 1u;
        const half8_t am = *reinterpret_cast<const half8_t*>(&sm.xm[bb][ar][8 * kq]);
        const half8_t bm = *reinterpret_cast<const half8_t*>(&sm.wm[bb][br][8 * kq]);
        const float16_t mins = mfma(am, bm, float16_t{});
        const float d = sm.dd[bb][br][0], dmin = sm.dd[bb][br][1];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          acc[r] = __builtin_fmaf(d, c[r], acc[r]);
          acc[r] = __builtin_fmaf(-dmin, mins[r], acc[r]);
        }
        c = float16_t{};
      }
    }
  };
  for (unsigned s = 0; s < n_stages; s += 2) {  // n_stages is even (k % 256 == 0)
    step(fa, s);
    step(fb, s + 1);
  }
  // Lane (row br, half kq) holds tokens 8 (r / 4) + 4 kq + r % 4 of the wave's 32.
  const unsigned n = n0 + br;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const unsigned tok = m0 + 32 * wt + 8 * (r / 4) + 4 * kq + r % 4;
    if (tok < p.n_tok && n < p.n_rows)
      p.y[std::size_t{tok} * p.ldy + n] = acc[r];
  }
}

// ---- Q4_K in 128 x 128 tiles (no reference counterpart) ----
// A workgroup computes 128 tokens x 128 rows, each wave a 64 x 64 quarter (2 x 2 MFMA blocks),
// so every operand read from LDS feeds two MFMAs instead of one. A stage's tiles are the 64 x 64
// fetch and store above done twice, at tile rows 0 and 64, and the store of stage s + 1 runs in
// the same step as the MFMAs of stage s, into the other buffer. Per output element the
// arithmetic is gemm_tile's in the same order, so both tile shapes give bit-identical results.
// The LDS (148 KiB) allows one workgroup per CU, against two for the 64 x 64 tiles, so these
// tiles pay only when they alone fill the chip (qgemm_big_tiles).
constexpr unsigned kBig = 128, kBigGroupTok = 4;

struct alignas(16) LdsBig {
  _Float16 x[2][kBig * kBK];
  _Float16 w[2][kBig * kBK];
  _Float16 xm[2][kBig][16];
  _Float16 wm[2][kBig][16];
  float dd[2][kBig][4];
};

__device__ __attribute__((always_inline)) inline void gemm_tile_big(const QGemmParams& p,
                                                                    LdsBig& sm, unsigned m0,
                                                                    unsigned n0) {
  constexpr QFormat F = QFormat::Q4K;
  const unsigned t = threadIdx.x, lane = t % 64, wave = t / 64;
  const unsigned wt = wave >> 1, wr = wave & 1u, kq = lane / 32;
  unsigned ar[2], br[2];  // the lane's token rows and weight rows in the tile, per MFMA block
#pragma unroll
  for (unsigned i = 0; i < 2; ++i) {
    ar[i] = 64 * wt + 32 * i + lane % 32;
    br[i] = 64 * wr + 32 * i + lane % 32;
  }
  const unsigned n_stages = p.k / kBK;
  bool tok_ok[2], row_ok[2];
#pragma unroll
  for (unsigned h = 0; h < 2; ++h) {
    tok_ok[h] = m0 + 64 * h + t / 4 < p.n_tok;
    row_ok[h] = n0 + 64 * h + t / 4 < p.n_rows;
  }
  auto fetch2 = [&](Fetch<F> (&f)[2], unsigned s) __attribute__((always_inline)) {
    f[0] = fetch<F>(p, n0, m0, s, t);
    f[1] = fetch<F>(p, n0 + 64, m0 + 64, s, t);
  };
  auto store2 = [&](const Fetch<F> (&f)[2], unsigned s) __attribute__((always_inline)) {
    store<F, LdsBig>(f[0], sm, s, t, tok_ok[0], row_ok[0], 0);
    store<F, LdsBig>(f[1], sm, s, t, tok_ok[1], row_ok[1], 64);
  };
  float16_t acc[2][2], c[2][2];
#pragma unroll
  for (unsigned i = 0; i < 2; ++i)
#pragma unroll
    for (unsigned j = 0; j < 2; ++j)
      acc[i][j] = c[i][j] = float16_t{};
  // Two register sets, even and odd stages, each requested two stages before its store.
  Fetch<F> fa[2], fb[2];
  fetch2(fa, 0);
  asm volatile("" : : : "memory");  // stage 0's loads are issued before stage 1's
  fetch2(fb, 1);
  store2(fa, 0);
  fetch2(fa, 2);
  auto step = [&](Fetch<F> (&fn)[2], unsigned s) __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    // Stage s complete in its buffer, and every wave done with the other one (stage s - 1).
    __syncthreads();
    // Also at the last stage (a re-read of it into the buffer and block parity nothing reads
    // again), so that the store shares one scheduling region with the MFMAs.
    store2(fn, s + 1);
    fetch2(fn, s + 3);  // past the last stage: re-reads it
    const unsigned buf = s & 1u;
#pragma unroll
    for (unsigned kk = 0; kk < kBK / 16; ++kk) {
      half8_t a[2], b[2];
#pragma unroll
      for (unsigned i = 0; i < 2; ++i) {
        a[i] = *reinterpret_cast<const half8_t*>(sm.x[buf] + chunk_at(ar[i], 2 * kk + kq));
        b[i] = *reinterpret_cast<const half8_t*>(sm.w[buf] + chunk_at(br[i], 2 * kk + kq));
      }
#pragma unroll
      for (unsigned i = 0; i < 2; ++i)
#pragma unroll
        for (unsigned j = 0; j < 2; ++j)
          c[i][j] = mfma(a[i], b[j], c[i][j]);
    }
    if (s % 2 == 1) {  // the block's last stage: its dmin m term, then its d scale
      const unsigned bb = (s / 2) & 1u;
#pragma unroll
      for (unsigned j = 0; j < 2; ++j) {
        const half8_t bm = *reinterpret_cast<const half8_t*>(&sm.wm[bb][br[j]][8 * kq]);
        const float d = sm.dd[bb][br[j]][0], dmin = sm.dd[bb][br[j]][1];
#pragma unroll
        for (unsigned i = 0; i < 2; ++i) {
          const half8_t am = *reinterpret_cast<const half8_t*>(&sm.xm[bb][ar[i]][8 * kq]);
          const float16_t mins = mfma(am, bm, float16_t{});
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            acc[i][j][r] = __builtin_fmaf(d, c[i][j][r], acc[i][j][r]);
            acc[i][j][r] = __builtin_fmaf(-dmin, mins[r], acc[i][j][r]);
          }
          c[i][j] = float16_t{};
        }
      }
    }
  };
  for (unsigned s = 0; s < n_stages; s += 2) {  // n_stages is even (k % 256 == 0)
    step(fb, s);
    step(fa, s + 1);
  }
  // Lane (row br[j], half kq) holds tokens 8 (r / 4) + 4 kq + r % 4 of token block i.
#pragma unroll
  for (unsigned j = 0; j < 2; ++j) {
    const unsigned n = n0 + br[j];
#pragma unroll
    for (unsigned i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const unsigned tok = m0 + 64 * wt + 32 * i + 8 * (r / 4) + 4 * kq + r % 4;
        if (tok < p.n_tok && n < p.n_rows)
          p.y[std::size_t{tok} * p.ldy + n] = acc[i][j][r];
      }
  }
}

// The 64 x 64 tiles [first, first + count), in grouped_tile's order.
template <QFormat F>
__device__ inline void gemm_small(const QGemmParams& p, unsigned first, unsigned count, Lds& sm) {
  const unsigned n_ttiles = (p.n_tok + kBM - 1) / kBM, n_rtiles = (p.n_rows + kBN - 1) / kBN;
  for (unsigned i = blockIdx.x; i < count; i += gridDim.x) {
    const unsigned tile = first + (gridDim.x == count ? xcd_tile(i, count) : i);
    unsigned ttile, rtile;
    grouped_tile(tile, n_ttiles, n_rtiles, ttile, rtile);
    gemm_tile<F, 0>(p, sm, ttile * kBM, rtile * kBN);
    __syncthreads();  // the next tile's first stores reuse buffer 0
  }
}

}  // namespace qgemm_detail

// Output tiles [first, first + count) of 64 tokens x 64 rows, in grouped_tile's order.
template <QFormat F>
__device__ void qgemm_op(const QGemmParams& p, unsigned first, unsigned count) {
  __shared__ qgemm_detail::Lds sm;
  qgemm_detail::gemm_small<F>(p, first, count, sm);
}

__host__ __device__ inline unsigned qgemm_tiles(unsigned n_rows, unsigned n_tok) {
  using namespace qgemm_detail;
  return (n_rows + kBN - 1) / kBN * ((n_tok + kBM - 1) / kBM);
}

template <QFormat F>
__global__ void __launch_bounds__(qgemm_detail::kThreads) qgemm_kernel(QGemmParams p) {
  qgemm_op<F>(p, 0, qgemm_tiles(p.n_rows, p.n_tok));
}

// Workgroups for a Q4_K product in 128 x 128 tiles, or 0 where 64 x 64 tiles are faster (at most
// 64 tokens, or fewer 128 x 128 tiles than the 256 CUs: the 64 x 64 kernel then runs two
// workgroups per CU). No reference counterpart: callers that know it launch
// qgemm_q4k_big_kernel on this many workgroups of 256 threads, else qgemm_kernel<Q4K>.
__host__ __device__ inline unsigned qgemm_big_tiles(unsigned n_rows, unsigned n_tok) {
  using namespace qgemm_detail;
  const unsigned tiles = (n_rows + kBig - 1) / kBig * ((n_tok + kBig - 1) / kBig);
  return n_tok > kBM && tiles >= 256 ? tiles : 0;
}

// The whole Q4_K product in 128 x 128 tiles (grid-stride over qgemm_big_tiles' tile count, in
// grouped_tile's order with groups of 4 token tiles). A template, so several translation units
// may include this header.
template <int = 0>
__global__ void __launch_bounds__(qgemm_detail::kThreads) qgemm_q4k_big_kernel(QGemmParams p) {
  using namespace qgemm_detail;
  __shared__ LdsBig sm;
  const unsigned n_ttiles = (p.n_tok + kBig - 1) / kBig, n_rtiles = (p.n_rows + kBig - 1) / kBig;
  const unsigned count = n_ttiles * n_rtiles;
  for (unsigned i = blockIdx.x; i < count; i += gridDim.x) {
    const unsigned tile = gridDim.x == count ? xcd_tile(i, count) : i;
    unsigned ttile, rtile;
    grouped_tile<kBigGroupTok>(tile, n_ttiles, n_rtiles, ttile, rtile);
    gemm_tile_big(p, sm, ttile * kBig, rtile * kBig);
    __syncthreads();  // the next tile's first stores reuse buffer 0
  }
}

}  // namespace miso::kernels
