#pragma once

// Q4_K GEMV y = W x for MI355X (gfx950 / CDNA4): the decode-time projections on either side of
// the attention (attn_q 2048 -> 8192, attn_k 2048 -> 512, attn_output 4096 -> 2048 are Q4_K in the
// engine's model). The interface is miso's kernels/q4k_gemv.hpp -- ActFormat, Q4kGemvParams,
// q4k_gemv_op<A, K, kBlock, kRows>(params, first, count, logical_block, logical_grid) and
// q4k_gemv_kernel<A, K, kBlock, kRows> keep their names, fields and template parameters, so the
// engine's launches (src/engine/weights.hip:248-279) and tests/test_q4k_gemv.hip compile against
// this header. The work decomposition and the arithmetic are this file's own.
//
// Weights are Q4_K "r1" blocks (src/repack.hpp:14-19): 144 bytes per 256 weights -- f16 d and
// dmin, then per nibble group j = 0..3 the 24-bit field sc[2j] | m[2j] << 6 | sc[2j+1] << 12 |
// m[2j+1] << 18 at byte 4 + 3j, then 4 x 32 nibble bytes: byte i of group j holds weight 64j + i
// (sub-block 2j) in its low nibble and weight 64j + 32 + i (sub-block 2j + 1) in its high nibble.
// w = d sc q - dmin m.
//
// Decomposition: the unit of work is one nibble group of one row (64 weights; its 32 nibble bytes
// and its block's 16-byte header). A lane keeps the same group position in every row it visits,
// so it reads its 64 activations once and holds them in registers. K / 64 groups per row are
// spread over a 32-lane half-wave (K = 2048: two rows per wave pass) or the whole wave (K >= 4096;
// K = 8192 gives each lane two groups). A wave's step is kRows passes of consecutive rows, one
// contiguous slab of weights: the wave streams it into its own LDS slab with
// global_load_lds_dwordx4 (1 KiB per instruction, every lane 16 consecutive bytes, so each
// instruction is one fully used run of cache lines and the bytes in flight cost no VGPRs); the
// workgroup meanwhile converts the activations once into LDS, and each lane then reads its group's
// activations and its units out of LDS. The lanes of a row combine with DPP and a permlane swap.
//
// Arithmetic (Fp16): each nibble pair is placed as the f16 integer 1024 + q (low nibble) or
// 1024 + 16 q (high nibble) by OR-ing it under the exponent of 1024 (the fast int4 -> f16 convert
// of Kim et al., "Who Says Elephants Can't Run", 2022), and one v_pk_fma_f16 turns that into q sc
// exactly (q sc <= 945; fused, so the intermediate never rounds). v_dot2_f32_f16 then accumulates
// sc q x in f32 over the whole group: the products are exact and one d per group scales the sum.
// Pairs are consecutive weights (v_perm_b32 spreads bytes 2i, 2i + 1 into the two halves), so the
// activations sit in natural order. The dmin m term uses the sum of the rounded activations of
// each sub-block. Int8: per-32 absmax activations (code = rint(x 127 / absmax)) meet the nibbles
// in v_dot4_i32_i8, one i32 chain per sub-block.

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
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr unsigned kBlockBytes = 144;

// Row geometry for K: `groups` nibble groups per row over `lanes` lanes (`per_lane` each); `rows`
// rows share one wave pass.
template <unsigned K>
struct Geometry {
  static_assert(K % 2048 == 0 && K <= 8192, "K is 2048, 4096 or 8192");
  static constexpr unsigned groups = K / 64;
  static constexpr unsigned lanes = groups < 64 ? groups : 64;
  static constexpr unsigned per_lane = groups / lanes;
  static constexpr unsigned rows = 64 / lanes;
  static constexpr std::size_t row_bytes = std::size_t{K} / 256 * kBlockBytes;
};

// Bytes 2i and 2i + 1 of w (i = 0, 1) in the low bytes of the two 16-bit halves.
__device__ __attribute__((always_inline)) inline unsigned spread_bytes(unsigned w, int i) {
  return __builtin_amdgcn_perm(0u, w, i == 0 ? 0x0C010C00u : 0x0C030C02u);
}

__device__ __attribute__((always_inline)) inline half2_t splat(float v) {
  return half2_t{static_cast<_Float16>(v), static_cast<_Float16>(v)};
}

// (v & mask) | bits in one v_and_or_b32 (the mask in an SGPR; gfx9 VOP3 takes no literal).
__device__ __attribute__((always_inline)) inline unsigned and_or(unsigned v, unsigned mask,
                                                                 unsigned bits) {
  unsigned r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(mask), "v"(bits));
  return r;
}

// The nibbles of v under mask, each placed under the exponent of 1024 (the f16 1024 + nibble, or
// 1024 + 16 nibble for a high mask), times s plus c: fused, so exact whenever the result is.
__device__ __attribute__((always_inline)) inline half2_t int_pair(unsigned v, unsigned mask,
                                                                  half2_t s, half2_t c) {
  return __builtin_elementwise_fma(cdna4::as_half2(and_or(v, mask, 0x64006400u)), s, c);
}

__device__ __attribute__((always_inline)) inline float f16_bits(unsigned h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(h)));
}

// The activations, converted once per workgroup into LDS: f16 values and per-32 sums of the
// rounded values (Fp16), or int8 codes with per-32 steps and sums (Int8). Four consecutive threads
// own one 32-element sub-block (8 elements each) and combine over their quad with DPP, so every
// value is the same whatever the workgroup size.
template <ActFormat A, unsigned K>
struct XStage;

template <unsigned K>
struct XStage<ActFormat::Fp16, K> {
  half2_t h[K / 2];
  float sum[K / 32];
};

template <unsigned K>
struct XStage<ActFormat::Int8, K> {
  unsigned q[K / 4];
  float step[K / 32], sum[K / 32];
};

// Sum / max over the 4 lanes of a quad.
__device__ __attribute__((always_inline)) inline float quad_sum(float v) {
  v += cdna4::dpp_mov<cdna4::kQuadXor1>(v);
  return v + cdna4::dpp_mov<cdna4::kQuadXor2>(v);
}
__device__ __attribute__((always_inline)) inline float quad_max(float v) {
  v = fmaxf(v, cdna4::dpp_mov<cdna4::kQuadXor1>(v));
  return fmaxf(v, cdna4::dpp_mov<cdna4::kQuadXor2>(v));
}

// The workgroup's activation area: the K floats as loaded, then (same bytes) their converted form.
template <ActFormat A, unsigned K>
union XArea {
  float f[K];
  XStage<A, K> s;
};

// Requests the K floats of x into xa.f with LDS DMA, instruction i (256 floats) from wave
// i % (kBlock / 64). Issued before the weights, so the weights' own waits cover it.
template <ActFormat A, unsigned K, int kBlock>
__device__ __attribute__((always_inline)) inline void issue_x(const float* x, XArea<A, K>& xa,
                                                              unsigned wave, unsigned lane) {
  const unsigned base = cdna4::lds_offset(xa.f);
  for (unsigned i = wave; i < K / 256; i += kBlock / 64)
    cdna4::lds_load16(x + 256 * i + 4 * lane, base + 1024 * i);
}

// Converts xa.f in place with the kBlock threads of the workgroup, once every wave's share has
// landed (each wave waits for its own DMA before calling). Thread t owns the 8-element slices
// 8 (t + kBlock s); a quad of threads covers one sub-block.
template <ActFormat A, unsigned K, int kBlock>
__device__ inline void convert_x(XArea<A, K>& xa) {
  constexpr unsigned kSlices = (K + 8 * kBlock - 1) / (8 * kBlock);
  static_assert(kSlices <= 4, "at most 32 activations per thread (K <= 32 kBlock)");
  const half2_t one{static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  float4 v[kSlices][2];
  __syncthreads();
#pragma unroll
  for (unsigned sl = 0; sl < kSlices; ++sl) {
    const unsigned e = 8 * (threadIdx.x + kBlock * sl);
    if (e < K) {
      v[sl][0] = *reinterpret_cast<const float4*>(&xa.f[e]);
      v[sl][1] = *reinterpret_cast<const float4*>(&xa.f[e + 4]);
    }
  }
  __syncthreads();  // every float is read before the converted form overwrites the area
#pragma unroll
  for (unsigned sl = 0; sl < kSlices; ++sl) {
    // Whole quads drop out together (K is a multiple of 32), so the quad DPP stays in-quad.
    const unsigned e = 8 * (threadIdx.x + kBlock * sl);
    if (e >= K)
      break;
    const float4 a = v[sl][0], b = v[sl][1];
    if constexpr (A == ActFormat::Fp16) {
      const half2_t h[4] = {half2_t{static_cast<_Float16>(a.x), static_cast<_Float16>(a.y)},
                            half2_t{static_cast<_Float16>(a.z), static_cast<_Float16>(a.w)},
                            half2_t{static_cast<_Float16>(b.x), static_cast<_Float16>(b.y)},
                            half2_t{static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)}};
      float part = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part = __builtin_amdgcn_fdot2(h[i], one, part, false);
      const float sum = quad_sum(part);
      *reinterpret_cast<u32x4*>(&xa.s.h[e / 2]) =
          u32x4{cdna4::as_uint(h[0]), cdna4::as_uint(h[1]), cdna4::as_uint(h[2]),
                cdna4::as_uint(h[3])};
      if ((threadIdx.x & 3u) == 0)
        xa.s.sum[e / 32] = sum;
    } else {
      const float f[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      float amax = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        amax = fmaxf(amax, __builtin_fabsf(f[i]));
      amax = quad_max(amax);
      const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
      unsigned word[2] = {0u, 0u};
      int total = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        int c = static_cast<int>(__builtin_rintf(f[i] * inv));
        c = c > 127 ? 127 : c < -127 ? -127 : c;
        total += c;
        word[i / 4] |= (static_cast<unsigned>(c) & 0xFFu) << (8 * (i % 4));
      }
      const float step = amax * (1.0f / 127.0f);
      const float codes = quad_sum(static_cast<float>(total));  // |sum| <= 4064: exact
      *reinterpret_cast<uint2*>(&xa.s.q[e / 4]) = uint2{word[0], word[1]};
      if ((threadIdx.x & 3u) == 0) {
        xa.s.step[e / 32] = step;
        xa.s.sum[e / 32] = step * codes;
      }
    }
  }
  __syncthreads();
}

// The lane's activations for one group position: sub-block lo (elements 0..31 of the group) and
// hi (32..63).
template <ActFormat A>
struct GroupX;

template <>
struct GroupX<ActFormat::Fp16> {
  half2_t lo[16], hi[16];  // (x[2i], x[2i + 1]) rounded to f16
  float sum_lo, sum_hi;    // sums of the rounded values
};

template <>
struct GroupX<ActFormat::Int8> {
  unsigned lo[8], hi[8];   // int8 codes, four per word, natural order
  float step_lo, step_hi;  // x ~ step * code
  float sum_lo, sum_hi;    // step * sum of the codes
};

// Activations of row group g (elements 64 g .. 64 g + 63) out of the staged copy.
template <ActFormat A, unsigned K>
__device__ inline GroupX<A> read_x(const XStage<A, K>& xs, unsigned g) {
  GroupX<A> r;
  if constexpr (A == ActFormat::Fp16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      r.lo[i] = xs.h[32 * g + i];
      r.hi[i] = xs.h[32 * g + 16 + i];
    }
    r.sum_lo = xs.sum[2 * g];
    r.sum_hi = xs.sum[2 * g + 1];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      r.lo[i] = xs.q[16 * g + i];
      r.hi[i] = xs.q[16 * g + 8 + i];
    }
    r.step_lo = xs.step[2 * g];
    r.step_hi = xs.step[2 * g + 1];
    r.sum_lo = xs.sum[2 * g];
    r.sum_hi = xs.sum[2 * g + 1];
  }
  return r;
}

// One unit: the block header and the group's 32 nibble bytes.
struct Unit {
  u32x4 head;
  u32x4 nib[2];
};

// Unit g of a row held in LDS at row (16-byte aligned).
__device__ __attribute__((always_inline)) inline Unit read_unit(const std::uint8_t* row,
                                                                unsigned g) {
  const std::uint8_t* blk = row + kBlockBytes * (g >> 2);
  const std::uint8_t* nib = blk + 16 + 32 * (g & 3u);
  Unit u;
  u.head = *reinterpret_cast<const u32x4*>(blk);
  u.nib[0] = *reinterpret_cast<const u32x4*>(nib);
  u.nib[1] = *reinterpret_cast<const u32x4*>(nib + 16);
  return u;
}

// A wave's weight slab: kPasses passes of kPassRows rows of kRowBytes bytes, moved by `instr` DMA
// instructions of 1 KiB; pass k can be read once the first ready(k) of them have landed.
template <unsigned kRowBytes, unsigned kPassRows, int kPasses>
struct Slab {
  static constexpr unsigned bytes = kRowBytes * kPassRows * kPasses;
  static constexpr unsigned instr = (bytes + 1023) / 1024;
  static constexpr unsigned alloc = instr * 1024;
  static_assert(instr < 64, "the slab's DMA count fits vmcnt");
  static constexpr unsigned ready(int k) {
    return ((k + 1) * kPassRows * kRowBytes + 1023) / 1024;
  }
};

// Waits until pass k of slab S (k < kPasses, a constant once the pass loop is unrolled) has landed.
template <class S, int kPasses, int c = 0>
__device__ __attribute__((always_inline)) inline void wait_pass(int k) {
  if constexpr (c < kPasses) {
    if (k == c)
      cdna4::wait_vmcnt<S::instr - S::ready(c)>();
    else
      wait_pass<S, kPasses, c + 1>(k);
  }
}

// Streams the first n bytes of src (16 <= n <= kInstr KiB, a multiple of 16) into a wave's slab at
// LDS byte address lds (wave-uniform): instruction i moves bytes 1024 i .. 1024 i + 1023, lane l
// the 16 at 1024 i + 16 l. Lanes past n re-read src's last 16 bytes into slab bytes nobody reads,
// so every instruction is always issued and the waits can count them. Non-temporal: each weight
// is read once.
template <unsigned kInstr>
__device__ __attribute__((always_inline)) inline void stage_slab(const std::uint8_t* src,
                                                                 unsigned lds, unsigned n,
                                                                 unsigned lane) {
#pragma unroll
  for (unsigned i = 0; i < kInstr; ++i) {
    const unsigned at = 1024 * i + 16 * lane;
    cdna4::lds_load16_nt(src + (at < n ? at : n - 16), lds + 1024 * i);
  }
}

__device__ __attribute__((always_inline)) inline void wait_lds_reads() {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
}

// The 24-bit scale field of group j: bits 24 j .. 24 j + 23 of header bytes 4..15.
__device__ __attribute__((always_inline)) inline unsigned scale_field(const u32x4& h, unsigned j) {
  const std::uint64_t a = static_cast<std::uint64_t>(h.z) << 32 | h.y;
  const std::uint64_t b = static_cast<std::uint64_t>(h.w) << 32 | h.z;
  const std::uint64_t v = j < 2 ? a >> (24 * j) : b >> (24 * j - 32);
  return static_cast<unsigned>(v) & 0xFFFFFFu;
}

template <ActFormat A>
__device__ __attribute__((always_inline)) inline float unit_dot(const Unit& u, unsigned j,
                                                                const GroupX<A>& x) {
  const unsigned f = scale_field(u.head, j);
  const unsigned sc_lo = f & 63u, m_lo = (f >> 6) & 63u;
  const unsigned sc_hi = (f >> 12) & 63u, m_hi = f >> 18;
  const float d = f16_bits(u.head.x & 0xFFFFu), dmin = f16_bits(u.head.x >> 16);
  const unsigned w[8] = {u.nib[0].x, u.nib[0].y, u.nib[0].z, u.nib[0].w,
                         u.nib[1].x, u.nib[1].y, u.nib[1].z, u.nib[1].w};
  const float mins = dmin * (static_cast<float>(m_lo) * x.sum_lo +
                             static_cast<float>(m_hi) * x.sum_hi);
  if constexpr (A == ActFormat::Fp16) {
    // Low nibbles: (1024 + q) sc - 1024 sc; high nibbles: (1024 + 16 q) sc / 16 - 64 sc.
    const half2_t s_lo = splat(static_cast<float>(sc_lo));
    const half2_t c_lo = splat(-1024.0f * static_cast<float>(sc_lo));
    const half2_t s_hi = splat(static_cast<float>(sc_hi) * 0.0625f);
    const half2_t c_hi = splat(-64.0f * static_cast<float>(sc_hi));
    float acc_lo = 0.0f, acc_hi = 0.0f;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const unsigned b = spread_bytes(w[t], i);
        acc_lo = __builtin_amdgcn_fdot2(int_pair(b, 0x000F000Fu, s_lo, c_lo), x.lo[2 * t + i],
                                        acc_lo, false);
        acc_hi = __builtin_amdgcn_fdot2(int_pair(b, 0x00F000F0u, s_hi, c_hi), x.hi[2 * t + i],
                                        acc_hi, false);
      }
    }
    return d * (acc_lo + acc_hi) - mins;
  } else {
    int acc_lo = 0, acc_hi = 0;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      acc_lo = __builtin_amdgcn_sdot4(static_cast<int>(w[t] & 0x0F0F0F0Fu),
                                      static_cast<int>(x.lo[t]), acc_lo, false);
      acc_hi = __builtin_amdgcn_sdot4(static_cast<int>((w[t] >> 4) & 0x0F0F0F0Fu),
                                      static_cast<int>(x.hi[t]), acc_hi, false);
    }
    return d * (static_cast<float>(sc_lo) * x.step_lo * static_cast<float>(acc_lo) +
                static_cast<float>(sc_hi) * x.step_hi * static_cast<float>(acc_hi)) -
           mins;
  }
}

// Sum over the kLanes consecutive lanes (16, 32 or 64) holding one row, in every one of them.
template <unsigned kLanes>
__device__ __attribute__((always_inline)) inline float row_sum(float v) {
  using namespace cdna4;
  static_assert(kLanes == 16 || kLanes == 32 || kLanes == 64, "row lane count");
  v += dpp_mov<kQuadXor1>(v);
  v += dpp_mov<kQuadXor2>(v);
  v += dpp_mov<kRowHalfMirror>(v);
  v += dpp_mov<kRowMirror>(v);
  if constexpr (kLanes >= 32)
    v = sum_xor16(v);
  if constexpr (kLanes == 64)
    v = sum_xor32(v);
  return v;
}

}  // namespace q4k_gemv_detail

// Rows a wave covers per step: kRows passes of Geometry<K>::rows rows.
template <unsigned K, int kRows>
__host__ __device__ constexpr unsigned q4k_gemv_wave_rows() {
  return q4k_gemv_detail::Geometry<K>::rows * static_cast<unsigned>(kRows);
}

// Rows [first, first + count) over logical_grid workgroups of kBlock threads (fused callers pass
// their own block index and grid; K <= 32 kBlock). Each wave takes q4k_gemv_wave_rows<K, kRows>()
// consecutive rows per step and strides by the number of waves; each next slab is requested as
// soon as the current one has been read out of LDS.
template <ActFormat A, unsigned K, int kBlock, int kRows = 1>
__device__ void q4k_gemv_op(const Q4kGemvParams& p, unsigned first, unsigned count,
                            unsigned logical_block = blockIdx.x,
                            unsigned logical_grid = gridDim.x) {
  using namespace q4k_gemv_detail;
  using G = Geometry<K>;
  using S = Slab<G::row_bytes, G::rows, kRows>;
  static_assert(kBlock % 64 == 0 && kRows >= 1, "whole waves, at least one pass");
  constexpr unsigned kStep = q4k_gemv_wave_rows<K, kRows>();
  __shared__ __attribute__((aligned(16))) std::uint8_t slab[kBlock / 64][S::alloc];
  __shared__ __attribute__((aligned(16))) XArea<A, K> x_lds;
  const unsigned lane = threadIdx.x % 64;
  const unsigned wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const unsigned wave = logical_block * (kBlock / 64) + wv;
  const unsigned waves = logical_grid * (kBlock / 64);
  const unsigned slot = lane % G::lanes, sub = lane / G::lanes;
  const unsigned j = slot & 3u;  // the lane's group index inside its blocks (lanes % 4 == 0)
  const unsigned end = first + count;
  const std::uint8_t* mine = slab[wv];
  const unsigned mine_lds = cdna4::lds_offset(mine);
  auto issue = [&](unsigned r0) __attribute__((always_inline)) {
    const unsigned rows = end - r0 < kStep ? end - r0 : kStep;
    stage_slab<S::instr>(p.w + std::size_t{r0} * G::row_bytes, mine_lds,
                         rows * static_cast<unsigned>(G::row_bytes), lane);
  };

  // Activations first, then the first slab; the wait for everything but the slab covers the
  // activations, and each pass below waits only for the slab instructions holding its rows.
  issue_x<A, K, kBlock>(p.x, x_lds, wv, lane);
  unsigned r0 = first + wave * kStep;
  if (r0 < end) {
    issue(r0);
    cdna4::wait_vmcnt<S::instr>();
  } else {
    cdna4::wait_vmcnt<0>();
  }
  convert_x<A, K, kBlock>(x_lds);
  GroupX<A> xs[G::per_lane];
#pragma unroll
  for (unsigned v = 0; v < G::per_lane; ++v)
    xs[v] = read_x<A, K>(x_lds.s, slot + G::lanes * v);

  for (; r0 < end; r0 += waves * kStep) {
    // Rows past `end` read stale slab bytes; their sums are never stored.
    float val[kRows];
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      wait_pass<S, kRows>(k);
      val[k] = 0.0f;
#pragma unroll
      for (unsigned v = 0; v < G::per_lane; ++v)
        val[k] += unit_dot<A>(read_unit(mine + (G::rows * k + sub) * G::row_bytes,
                                        slot + G::lanes * v),
                              j, xs[v]);
    }
    if (r0 + waves * kStep < end) {
      wait_lds_reads();
      issue(r0 + waves * kStep);
    }
#pragma unroll
    for (int k = 0; k < kRows; ++k) {
      const float s = row_sum<G::lanes>(val[k]);
      const unsigned r = r0 + G::rows * k + sub;
      if (slot == 0 && r < end)
        p.y[r] = s;
    }
  }
}

template <ActFormat A, unsigned K, int kBlock, int kRows = 1>
__global__ void __launch_bounds__(kBlock) q4k_gemv_kernel(Q4kGemvParams p) {
  q4k_gemv_op<A, K, kBlock, kRows>(p, 0, p.n_rows);
}

}  // namespace miso::kernels
