#pragma once

// Q6_K GEMV y = W x for MI355X (gfx950 / CDNA4), f16 activations: the attention's attn_v
// projection (2048 -> 512, Q6_K in the engine's model). The interface is miso's
// kernels/q6k_gemv.hpp -- Q6kGemvParams, q6k_gemv_op<K, kBlock, kRows>(params, first, count,
// logical_block, logical_grid) and q6k_gemv_kernel<K, kBlock, kRows> keep their names, fields and
// template parameters; the decomposition and the arithmetic are this file's own, the same scheme
// as the Q4_K GEMV beside it.
//
// Weights are Q6_K "r1" rows (src/repack.hpp:25-28): a row of nb = K / 256 GGUF blocks stored as
// [ql: nb x 128][qh: nb x 64][scales: nb x 16 int8][d: nb x 2 f16], zero-padded to 16 bytes.
// Element e of half h (e < 128) of block b has the 6-bit code (ql[b][64 h + e % 64] >> 4 (e / 64)
// & 15) | (qh[b][32 h + e % 32] >> 2 (e / 32) & 3) << 4 and the weight d sc[b][8 h + e / 16]
// (code - 32).
//
// Decomposition: the unit of work is 64 weights of one row -- 32 ql bytes of a block half, whose
// low nibbles and high nibbles are two 32-element sets, with the half's 32 qh bytes, 4 scales and
// d. A lane keeps the same unit position in every row, so it reads its 64 activations once. K / 64
// units per row over 32 lanes (K = 2048: two rows per wave pass) or the whole wave (K >= 4096;
// K = 8192 gives each lane two units). A wave's step (kRows passes, one
// contiguous run of rows) is streamed into the wave's LDS slab with global_load_lds_dwordx4 while
// the workgroup converts the activations into LDS once, as in the Q4_K GEMV.
//
// Arithmetic: a code pair of consecutive elements becomes the f16 integer 1024 + c or 1024 + 16 c
// (the fast int -> f16 convert of Kim et al., 2022), then c - 32 or 16 (c - 32) exactly with one
// v_pk_add_f16; v_dot2_f32_f16 accumulates it times x over each 16-element scale group in f32
// (exact products), and the lane sums sc (or sc / 16) times its four group chains before one
// multiply by d. (c - 32) sc is not folded into the f16 weight: it can exceed 2048 and would round.

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

// Row geometry for K: K / 64 units per row (a unit is half c of the 64-element element sets of one
// block half, see below) over `lanes` lanes (`per_lane` each); `rows` rows share one wave pass.
template <unsigned K>
struct Geometry {
  static_assert(K % 2048 == 0 && K <= 8192, "K is 2048, 4096 or 8192");
  static constexpr unsigned nb = K / 256;
  static constexpr unsigned units = K / 64;
  static constexpr unsigned lanes = units < 64 ? units : 64;
  static constexpr unsigned per_lane = units / lanes;
  static constexpr unsigned rows = 64 / lanes;
  static constexpr std::size_t row_bytes = (std::size_t{nb} * 210 + 15) / 16 * 16;
};

// Unit u of a row: block u / 4, half h = u / 2 % 2, part c = u % 2. It covers ql bytes 32c .. 32c +
// 31 of the half, i.e. elements 32c + i (low nibbles, scale groups 2c, 2c + 1) and 64 + 32c + i
// (high nibbles, scale groups 4 + 2c, 5 + 2c), i < 32, whose top bits sit at bit 2c (low) and
// 2c + 4 (high) of the half's qh byte i.
struct UnitX {
  half2_t lo[16], hi[16];  // consecutive f16 pairs of the two element sets
};

template <unsigned K>
__device__ inline UnitX read_x(const q4k_gemv_detail::XStage<ActFormat::Fp16, K>& xs, unsigned u) {
  const unsigned e = 128 * (u >> 1) + 32 * (u & 1u);  // first element of the low set
  UnitX r;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    r.lo[i] = xs.h[e / 2 + i];
    r.hi[i] = xs.h[(e + 64) / 2 + i];
  }
  return r;
}

struct Unit {
  u32x4 ql[2], qh[2];
  unsigned sc_lo, sc_hi;  // int8 scales of groups 2c, 2c + 1 / 4 + 2c, 5 + 2c in bytes 0, 1
  unsigned d_bits;        // f16 d in the low 16 bits
};

// Unit u of a row held in LDS at row.
template <unsigned K>
__device__ __attribute__((always_inline)) inline Unit read_unit(const std::uint8_t* row,
                                                                unsigned u) {
  using G = Geometry<K>;
  const unsigned b = u >> 2, h = (u >> 1) & 1u, c = u & 1u;
  const std::uint8_t* ql = row + 128 * b + 64 * h + 32 * c;
  const std::uint8_t* qh = row + G::nb * 128 + 64 * b + 32 * h;
  const std::uint8_t* sc = row + G::nb * 192 + 16 * b + 8 * h + 2 * c;
  Unit r;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    r.ql[i] = *reinterpret_cast<const u32x4*>(ql + 16 * i);
    r.qh[i] = *reinterpret_cast<const u32x4*>(qh + 16 * i);
  }
  r.sc_lo = *reinterpret_cast<const unsigned short*>(sc);
  r.sc_hi = *reinterpret_cast<const unsigned short*>(sc + 4);
  r.d_bits = *reinterpret_cast<const unsigned short*>(row + G::nb * 208 + 2 * b);
  return r;
}

__device__ __attribute__((always_inline)) inline unsigned word(const u32x4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// The codes of bytes 2i, 2i + 1 of ql word l / qh word q, for the low-nibble element set (top
// bits at bit s of the qh byte, s = 0 or 2) and the high-nibble set (top bits at s + 4). One shift
// of the spread qh bytes puts the low set's top bits at bits 4-5 and the high set's at 8-9, under
// the high nibbles; nested v_and_or_b32 then build the f16 1024 + c (low set) and 1024 + 16 c
// (high set), and one v_pk_add_f16 each leaves c - 32 and 16 (c - 32), exactly.
struct CodePairs {
  half2_t lo, hi16;
};

__device__ __attribute__((always_inline)) inline CodePairs code_pairs(unsigned l, unsigned q, int i,
                                                                      unsigned s) {
  using q4k_gemv_detail::and_or;
  const unsigned lb = q4k_gemv_detail::spread_bytes(l, i);
  const unsigned t = q4k_gemv_detail::spread_bytes(q, i) << (4 - s);
  const unsigned lo = and_or(lb, 0x000F000Fu, and_or(t, 0x00300030u, 0x64006400u));
  const unsigned hi = and_or(lb, 0x00F000F0u, and_or(t, 0x03000300u, 0x64006400u));
  const _Float16 b_lo = static_cast<_Float16>(-1056.0f);  // -(1024 + 32)
  const _Float16 b_hi = static_cast<_Float16>(-1536.0f);  // -(1024 + 16 * 32)
  return {cdna4::as_half2(lo) + half2_t{b_lo, b_lo}, cdna4::as_half2(hi) + half2_t{b_hi, b_hi}};
}

// Unit u's sum of w x: two scale groups per element set, each a v_dot2_f32_f16 chain of 8 pairs.
__device__ __attribute__((always_inline)) inline float unit_dot(const Unit& u, unsigned c,
                                                                const UnitX& x) {
  float chain[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // low set groups 0, 1; high set groups 0, 1 (x16)
#pragma unroll
  for (int t = 0; t < 8; ++t) {  // ql word t: elements 4t .. 4t + 3 of each set
    const unsigned l = word(u.ql[t >> 2], t & 3);
    const unsigned q = word(u.qh[t >> 2], t & 3);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const CodePairs p = code_pairs(l, q, i, 2 * c);
      chain[t >> 2] = __builtin_amdgcn_fdot2(p.lo, x.lo[2 * t + i], chain[t >> 2], false);
      chain[2 + (t >> 2)] =
          __builtin_amdgcn_fdot2(p.hi16, x.hi[2 * t + i], chain[2 + (t >> 2)], false);
    }
  }
  auto sc = [](unsigned w, int b) {
    return static_cast<float>(static_cast<signed char>((w >> (8 * b)) & 0xFFu));
  };
  float acc = sc(u.sc_lo, 0) * chain[0];
  acc = __builtin_fmaf(sc(u.sc_lo, 1), chain[1], acc);
  acc = __builtin_fmaf(sc(u.sc_hi, 0) * 0.0625f, chain[2], acc);
  acc = __builtin_fmaf(sc(u.sc_hi, 1) * 0.0625f, chain[3], acc);
  return q4k_gemv_detail::f16_bits(u.d_bits & 0xFFFFu) * acc;
}

}  // namespace q6k_gemv_detail

template <unsigned K, int kRows>
__host__ __device__ constexpr unsigned q6k_gemv_wave_rows() {
  return q6k_gemv_detail::Geometry<K>::rows * static_cast<unsigned>(kRows);
}

// Rows [first, first + count) over logical_grid workgroups of kBlock threads (K <= 32 kBlock); each
// wave takes q6k_gemv_wave_rows<K, kRows>() consecutive rows per step, the same pipeline as
// q4k_gemv_op.
template <unsigned K, int kBlock, int kRows = 1>
__device__ void q6k_gemv_op(const Q6kGemvParams& p, unsigned first, unsigned count,
                            unsigned logical_block = blockIdx.x,
                            unsigned logical_grid = gridDim.x) {
  using namespace q6k_gemv_detail;
  using q4k_gemv_detail::XArea;
  using G = Geometry<K>;
  using S = q4k_gemv_detail::Slab<G::row_bytes, G::rows, kRows>;
  static_assert(kBlock % 64 == 0 && kRows >= 1, "whole waves, at least one pass");
  constexpr unsigned kStep = q6k_gemv_wave_rows<K, kRows>();
  __shared__ __attribute__((aligned(16))) std::uint8_t slab[kBlock / 64][S::alloc];
  __shared__ __attribute__((aligned(16))) XArea<ActFormat::Fp16, K> x_lds;
  const unsigned lane = threadIdx.x % 64;
  const unsigned wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const unsigned wave = logical_block * (kBlock / 64) + wv;
  const unsigned waves = logical_grid * (kBlock / 64);
  const unsigned slot = lane % G::lanes, sub = lane / G::lanes;
  const unsigned end = first + count;
  const std::uint8_t* mine = slab[wv];
  const unsigned mine_lds = cdna4::lds_offset(mine);
  auto issue = [&](unsigned r0) __attribute__((always_inline)) {
    const unsigned rows = end - r0 < kStep ? end - r0 : kStep;
    q4k_gemv_detail::stage_slab<S::instr>(p.w + std::size_t{r0} * G::row_bytes, mine_lds,
                                          rows * static_cast<unsigned>(G::row_bytes), lane);
  };

  q4k_gemv_detail::issue_x<ActFormat::Fp16, K, kBlock>(p.x, x_lds, wv, lane);
  unsigned r0 = first + wave * kStep;
  if (r0 < end) {
    issue(r0);
    cdna4::wait_vmcnt<S::instr>();
  } else {
    cdna4::wait_vmcnt<0>();
  }
  q4k_gemv_detail::convert_x<ActFormat::Fp16, K, kBlock>(x_lds);
  UnitX xs[G::per_lane];
#pragma unroll
  for (unsigned v = 0; v < G::per_lane; ++v)
    xs[v] = read_x<K>(x_lds.s, slot + G::lanes * v);

  for (; r0 < end; r0 += waves * kStep) {
    float val[kRows];  // rows past `end` read stale slab bytes; their sums are never stored
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      q4k_gemv_detail::wait_pass<S, kRows>(k);
      val[k] = 0.0f;
#pragma unroll
      for (unsigned v = 0; v < G::per_lane; ++v) {
        const unsigned un = slot + G::lanes * v;
        val[k] += unit_dot(read_unit<K>(mine + (G::rows * k + sub) * G::row_bytes, un), un & 1u,
                           xs[v]);
      }
    }
    if (r0 + waves * kStep < end) {
      q4k_gemv_detail::wait_lds_reads();
      issue(r0 + waves * kStep);
    }
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const float s = q4k_gemv_detail::row_sum<G::lanes>(val[k]);
      const unsigned r = r0 + G::rows * k + sub;
      if (slot == 0 && r < end)
        p.y[r] = s;
    }
  }
}

template <unsigned K, int kBlock, int kRows = 1>
__global__ void __launch_bounds__(kBlock) q6k_gemv_kernel(Q6kGemvParams p) {
  q6k_gemv_op<K, kBlock, kRows>(p, 0, p.n_rows);
}

}  // namespace miso::kernels
