#pragma once

// Decode over an fp8 KV cache for MI355X (gfx950 / CDNA4). No reference counterpart: the
// reference's cache is f16 [kv_head][max_ctx][256] (src/engine/attention.hpp:35-41,
// kernels/attention_decode.hpp:26-27); this format halves the bytes a decode step streams.
//
// Format ("e4m3 rows"): row (KV head, position) is 256 one-byte OCP e4m3 codes (bias 7, no
// infinities, 0x7F / 0xFF NaN; the encoder never emits them) in k8 / v8 [2][max_ctx][256], and
// one f32 scale in k_scale / v_scale [2][max_ctx]. value[d] = scale * e4m3(code[d]). The scale is
// the power of two 2^(E - 7), E = floor(log2 max_d |x[d]|) (E = -100 for rows whose max is below
// 2^-100, zero rows included), so x / scale is exact and lies in (-256, 256): encoding is a
// round-to-nearest-even to 3 mantissa bits (subnormal step 2^-9) and never saturates. Inputs
// must be finite.
//
// Kernels:
//   attn_kv_fp8_encode_kernel<256>  f16 cache rows [pos0, pos0 + n) of both KV heads -> e4m3 rows
//   attn_prep_fp8_kernel<256>       attn_prep (RMSNorm + RoPE) appending the token as e4m3 rows
//   attn_prep_batch_fp8_kernel<256> the same for a batch of tokens (attn_prep_batch's layout)
//   attn_kv_fp8_widen_kernel<256>   e4m3 rows -> f16 rows, for the f16 prefill over an e4m3 cache
//   attn_split_fp8_kernel<256>      split-K partials over e4m3 rows on the matrix cores, at the
//                                   f16 split's precision, in the reference's partial layout;
//                                   attn_combine_kernel merges them unchanged.

#include "attention_decode.hpp"

namespace miso::kernels {

namespace fp8kv {

constexpr int kMinExp = -100;  // rows with max |x| < 2^-100 use E = -100

// Scale exponent E - 7 of a row whose largest magnitude is amax (finite, >= 0).
__device__ inline int scale_exponent(float amax) {
  const int e = static_cast<int>(__builtin_bit_cast(unsigned, amax) >> 23) - 127;
  return (e > kMinExp ? e : kMinExp) - 7;
}
__device__ inline float exp2i(int e) {  // 2^e for -126 <= e <= 127
  return __builtin_bit_cast(float, static_cast<unsigned>(e + 127) << 23);
}

// e4m3 code of y rounded to nearest even, |y| < 256.
__device__ inline unsigned encode(float y) {
  const float a = __builtin_fabsf(y);
  unsigned code;
  if (a < 0.015625f) {  // below 2^-6: subnormal codes 0..8 (8 is 2^-6, the smallest normal)
    code = static_cast<unsigned>(__builtin_rintf(a * 512.0f));
  } else {  // round the f32 mantissa to 3 bits, then rebias the exponent (127 -> 7)
    const unsigned b = __builtin_bit_cast(unsigned, a);
    code = ((b + 0x7FFFFu + ((b >> 20) & 1u)) >> 20) - (120u << 3);
  }
  return code | ((__builtin_bit_cast(unsigned, y) >> 24) & 0x80u);
}

// Two e4m3 codes (bytes 0, 1 or, for the _hi form, bytes 2, 3 of w) as an f16 pair, exactly
// (every e4m3 value is an f16 value). Inline assembly, so the compiler's model of the
// instruction's result lanes is not involved.
__device__ __attribute__((always_inline)) inline unsigned pair_lo(unsigned w) {
  unsigned r;
  asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, 1.0" : "=v"(r) : "v"(w));
  return r;
}
__device__ __attribute__((always_inline)) inline unsigned pair_hi(unsigned w) {
  unsigned r;
  asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, 1.0 op_sel:[1,0,0]" : "=v"(r) : "v"(w));
  return r;
}

// Block-wide max over the 256 threads (one value each); `red` holds 4 floats of LDS.
__device__ inline float block_max256(float v, float* red) {
  const float w = cdna4::wave_allmax(v);
  if ((threadIdx.x & 63u) == 0)
    red[threadIdx.x >> 6] = w;
  __syncthreads();
  const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();  // red is reused
  return m;
}

}  // namespace fp8kv

// ------------------------------------------------------------------------------------------------
// Encode: f16 cache rows -> e4m3 rows
// ------------------------------------------------------------------------------------------------

struct AttnKvFp8EncodeParams {
  const attn::half_t* k_cache;  // [2][max_ctx][256]
  const attn::half_t* v_cache;
  uint8_t* k8;                  // [2][max_ctx][256]
  uint8_t* v8;
  float* k_scale;               // [2][max_ctx]
  float* v_scale;
  unsigned pos0, n, max_ctx;
};

// One wave per row (4 per workgroup), lane i holding dimensions 4 i .. 4 i + 3; row r of the 4 n
// is (position pos0 + r / 4, KV head r / 2 % 2, K if r is even else V). Grid-stride.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_kv_fp8_encode_kernel(AttnKvFp8EncodeParams p) {
  static_assert(kBlock == 256, "four rows per workgroup");
  const unsigned lane = threadIdx.x & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (unsigned r = 4 * blockIdx.x + wave; r < 4 * p.n; r += 4 * gridDim.x) {
    const bool is_v = r & 1u;
    const unsigned kvh = (r >> 1) & 1u, pos = p.pos0 + (r >> 2);
    const std::size_t row = std::size_t{kvh} * p.max_ctx + pos;
    const attn::half_t* src = (is_v ? p.v_cache : p.k_cache) + row * attn::kDim + 4 * lane;
    const uint2 raw = *reinterpret_cast<const uint2*>(src);
    const cdna4::half2_t h0 = cdna4::as_half2(raw.x), h1 = cdna4::as_half2(raw.y);
    const float x[4] = {static_cast<float>(h0[0]), static_cast<float>(h0[1]),
                        static_cast<float>(h1[0]), static_cast<float>(h1[1])};
    float amax = fmaxf(fmaxf(__builtin_fabsf(x[0]), __builtin_fabsf(x[1])),
                       fmaxf(__builtin_fabsf(x[2]), __builtin_fabsf(x[3])));
    amax = cdna4::wave_allmax(amax);
    const int se = fp8kv::scale_exponent(amax);
    const float inv = fp8kv::exp2i(-se);
    unsigned packed = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      packed |= fp8kv::encode(x[i] * inv) << (8 * i);
    *reinterpret_cast<unsigned*>((is_v ? p.v8 : p.k8) + row * attn::kDim + 4 * lane) = packed;
    if (lane == 0)
      (is_v ? p.v_scale : p.k_scale)[row] = fp8kv::exp2i(se);
  }
}

// ------------------------------------------------------------------------------------------------
// Prep with an e4m3 append
// ------------------------------------------------------------------------------------------------

// AttnPrepParams with the f16 cache pointers replaced by the e4m3 rows and their scales.
struct AttnPrepFp8Params {
  const float* qg;
  const float* k;
  const float* v;
  const float* q_norm;
  const float* k_norm;
  const float* inv_freq;
  uint8_t* k8;       // [2][max_ctx][256]
  uint8_t* v8;
  float* k_scale;    // [2][max_ctx]
  float* v_scale;
  float* q;          // [16][256]
  unsigned pos, max_ctx;
  float eps;
};

// The query heads as attn_prep_head (same arithmetic, same q output); a KV head encodes its
// normalised, rotated K row and its V row at position pos.
template <int kBlock>
__device__ void attn_prep_fp8_head(const AttnPrepFp8Params& p, unsigned head) {
  static_assert(kBlock == attn::kDim, "one thread per dimension");
  __shared__ float wave_ss[kBlock / cdna4::kLanes];
  __shared__ float red[kBlock / cdna4::kLanes];
  const unsigned d = threadIdx.x;
  const float x = decode_detail::prep_value<kBlock>(p, head, wave_ss);
  if (head < static_cast<unsigned>(attn::kQHeads)) {
    p.q[head * attn::kDim + d] = x;
    return;  // uniform across the workgroup; prep_value leaves wave_ss free
  }
  const unsigned kvh = head - attn::kQHeads;
  const std::size_t row = std::size_t{kvh} * p.max_ctx + p.pos;
  const float v = p.v[kvh * attn::kDim + d];
  const int ke = fp8kv::scale_exponent(fp8kv::block_max256(__builtin_fabsf(x), red));
  const int ve = fp8kv::scale_exponent(fp8kv::block_max256(__builtin_fabsf(v), red));
  p.k8[row * attn::kDim + d] = static_cast<uint8_t>(fp8kv::encode(x * fp8kv::exp2i(-ke)));
  p.v8[row * attn::kDim + d] = static_cast<uint8_t>(fp8kv::encode(v * fp8kv::exp2i(-ve)));
  if (d == 0) {
    p.k_scale[row] = fp8kv::exp2i(ke);
    p.v_scale[row] = fp8kv::exp2i(ve);
  }
}

// 18 heads, one workgroup each (grid-stride), as attn_prep_kernel: grid 18 x 256.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prep_fp8_kernel(AttnPrepFp8Params p) {
  for (unsigned head = blockIdx.x; head < attn::kQHeads + attn::kKvHeads; head += gridDim.x)
    attn_prep_fp8_head<kBlock>(p, head);
}

// ------------------------------------------------------------------------------------------------
// Batched prep with an e4m3 append (the counterpart of attn_prep_batch_kernel,
// kernels/attention_prefill.hpp:20-40)
// ------------------------------------------------------------------------------------------------

// Token t of the batch: tok0 with qg / k / v advanced by t proj_stride floats, q by t 16 x 256
// floats and the position by t (AttnPrepBatchParams over e4m3 rows).
struct AttnPrepBatchFp8Params {
  AttnPrepFp8Params tok0;
  unsigned n, proj_stride;
};

// Items [0, 18 n) token-major, one workgroup each (grid-stride): attn_prep_fp8_head of token
// item / 18, head item % 18, so every row equals the one attn_prep_fp8_kernel writes for it.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prep_batch_fp8_kernel(AttnPrepBatchFp8Params p) {
  constexpr unsigned kHeads = attn::kQHeads + attn::kKvHeads;
  for (unsigned item = blockIdx.x; item < p.n * kHeads; item += gridDim.x) {
    const unsigned t = item / kHeads, head = item % kHeads;
    AttnPrepFp8Params one = p.tok0;
    one.qg += std::size_t{t} * p.proj_stride;
    one.k += std::size_t{t} * p.proj_stride;
    one.v += std::size_t{t} * p.proj_stride;
    one.q += std::size_t{t} * attn::kQHeads * attn::kDim;
    one.pos += t;
    attn_prep_fp8_head<kBlock>(one, head);
  }
}

// ------------------------------------------------------------------------------------------------
// Widening e4m3 rows to f16 (prefill over an e4m3 cache)
// ------------------------------------------------------------------------------------------------

// The causal prefill is bound by its MFMAs, which take f16 operands: over an e4m3 cache the
// rows a chunk attends to are widened once into an f16 workspace and the f16 prefill runs on it
// (the widening moves 3 bytes per element, microseconds against the milliseconds of the MFMAs).
// Rows [0, n) of both KV heads of the e4m3 cache (head stride max_ctx rows) go to the workspace
// [2][n][256] f16 (head stride n rows): value = scale e4m3(code), exact in f32, rounded to f16
// (RNE) after saturating at +-65504 -- only a row whose largest magnitude rounds to 2^16 at
// encoding (max |x| >= 63488) reaches that bound.
struct AttnKvFp8WidenParams {
  const uint8_t* k8;  // [2][max_ctx][256]
  const uint8_t* v8;
  const float* k_scale;  // [2][max_ctx]
  const float* v_scale;
  attn::half_t* k_out;  // [2][n][256]
  attn::half_t* v_out;
  unsigned n, max_ctx;
};

// One wave per row (4 per workgroup), lane i widening dimensions 4 i .. 4 i + 3; row r of the 4 n
// is (position r / 4, KV head r / 2 % 2, K if r is even else V). Grid-stride.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_kv_fp8_widen_kernel(AttnKvFp8WidenParams p) {
  static_assert(kBlock == 256, "four rows per workgroup");
  const unsigned lane = threadIdx.x & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (unsigned r = 4 * blockIdx.x + wave; r < 4 * p.n; r += 4 * gridDim.x) {
    const bool is_v = r & 1u;
    const unsigned kvh = (r >> 1) & 1u, pos = r >> 2;
    const std::size_t src = std::size_t{kvh} * p.max_ctx + pos;
    const std::size_t dst = std::size_t{kvh} * p.n + pos;
    const unsigned w = *reinterpret_cast<const unsigned*>((is_v ? p.v8 : p.k8) +
                                                          src * attn::kDim + 4 * lane);
    const float sc = (is_v ? p.v_scale : p.k_scale)[src];
    const cdna4::half2_t a = cdna4::as_half2(fp8kv::pair_lo(w));
    const cdna4::half2_t b = cdna4::as_half2(fp8kv::pair_hi(w));
    const float e[4] = {static_cast<float>(a[0]), static_cast<float>(a[1]),
                        static_cast<float>(b[0]), static_cast<float>(b[1])};
    _Float16 h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      h[i] = static_cast<_Float16>(fminf(fmaxf(e[i] * sc, -65504.0f), 65504.0f));
    *reinterpret_cast<uint2*>((is_v ? p.v_out : p.k_out) + dst * attn::kDim + 4 * lane) =
        __builtin_bit_cast(uint2, h);
  }
}

// ------------------------------------------------------------------------------------------------
// Split-K decode over e4m3 rows
// ------------------------------------------------------------------------------------------------

struct AttnSplitFp8Params {
  const float* q;        // [16][256]
  const uint8_t* k8;     // [2][max_ctx][256]
  const uint8_t* v8;
  const float* k_scale;  // [2][max_ctx]
  const float* v_scale;
  float* part_m;         // [2][n_splits][8], natural-log max of the scaled scores
  float* part_l;         // [2][n_splits][8]
  float* part_o;         // [2][n_splits][8][256]
  unsigned len, max_ctx, n_splits;
};

namespace decode_detail {

// ------------------------------------------------------------------------------------------------
// The split over e4m3 rows on the matrix cores, per-wave tiles (split_partial_waves' schedule and
// arithmetic over widened codes). Wave w takes the span's 32-key tiles w, w + 4, ...; a tile's
// codes (K and V, 8 KiB each) and row scales move by LDS-DMA into one of the wave's two stages,
// so the wave's next two tiles are in flight while it computes one. The codes widen to f16 in
// registers (every e4m3 value is an f16 value): K as the A operands of the score MFMAs against
// the (hi, lo) query pairs, each score then multiplied by its K row scale in f32; V read
// transposed (ds_read_b64_tr_b8) as the V^T operands. The numerators carry each row's V scale
// relative to a reference V scale R, the largest the wave has met in the item: O is kept
// relative to R (rescaled, exactly, when a tile brings a larger one) and multiplied by it at the
// end. So the arithmetic is the f16 path's (f32-precision query and numerators, f32 accumulation)
// on the rows the codes and scales define, and a common power-of-two factor on every V scale
// scales O exactly.
// ------------------------------------------------------------------------------------------------

// Wave w's stages: K codes at [0, 8192), V codes at [8192, 16384), row r at 256 r with 16-byte
// chunk c at position c ^ fp8_swz(r); the tile's K then V row scales.
struct alignas(1024) Fp8WaveShared {
  unsigned char codes[kWaves][2][16384];
  float scale[kWaves][2][64];
  float q[kGroup][attn::kDim];
};

// Chunk swizzle of tile row r: r % 16, with bit 3 flipped for rows 16-31. The A-operand K reads
// take one chunk of rows 16 kb + 0..15 (16 positions), the transposed V reads rows 4 g + j and
// 16 + 4 g + j together (8 positions apart).
__device__ __attribute__((always_inline)) inline unsigned fp8_swz(unsigned r) {
  return (r & 15u) ^ ((r >> 4 & 1u) << 3);
}

// Copy offsets of the two 16-row groups of a tile's codes: instruction i moves rows
// 16 grp + 4 i + lane / 16, chunk position lane % 16 (the lane's offset from the group's first row
// minus 1024 i, which the instruction offset adds).
__device__ __attribute__((always_inline)) inline void fp8_copy_offsets(unsigned (&off)[2][4],
                                                                      unsigned lane) {
#pragma unroll
  for (unsigned grp = 0; grp < 2; ++grp)
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
      const unsigned r = 16 * grp + 4 * i + (lane >> 4), pos = lane & 15u;
      off[grp][i] = (lane >> 4) * 256 + 16 * (pos ^ fp8_swz(r));
    }
}

// 8 copies of 1 KiB: rows 0-15 of the codes at xt to lds, rows 16-31 from xt + 4096 to lds + 4096.
// M0 is saved and restored.
__device__ __attribute__((always_inline)) inline void issue_codes32(const void* xt, const void* xt2,
                                                                   const unsigned (&off)[2][4],
                                                                   unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %11\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %9 nt\n\t"
      "global_load_lds_dwordx4 %2, %9 offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %3, %9 offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %4, %9 offset:3072 nt\n\t"
      "s_mov_b32 m0, %12\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %5, %10 nt\n\t"
      "global_load_lds_dwordx4 %6, %10 offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %7, %10 offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %8, %10 offset:3072 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off[0][0]), "v"(off[0][1]), "v"(off[0][2]), "v"(off[0][3]), "v"(off[1][0]),
        "v"(off[1][1]), "v"(off[1][2]), "v"(off[1][3]), "s"(xt), "s"(xt2), "s"(lds),
        "s"(lds + 4096u)
      : "memory");
}

// This wave's copy of the codes of the tile at key k0 (X: the KV head's K or V codes) into lds:
// 8 vector-memory instructions; rows past last_row read last_row (masked at use).
__device__ __attribute__((always_inline)) inline void issue_fp8_codes(const uint8_t* X,
                                                                     unsigned k0,
                                                                     unsigned last_row,
                                                                     unsigned lds,
                                                                     const unsigned (&off)[2][4],
                                                                     unsigned lane) {
  if (k0 + 31 <= last_row) {
    const uint8_t* base = reinterpret_cast<const uint8_t*>(
        uniform(reinterpret_cast<const attn::half_t*>(X + std::size_t{k0} * attn::kDim)));
    issue_codes32(base, base + 4096, off, lds);
  } else {
#pragma unroll
    for (unsigned i = 0; i < 8; ++i) {
      const unsigned r = 4 * i + (lane >> 4), pos = lane & 15u;
      const unsigned row = k0 + r <= last_row ? k0 + r : last_row;
      cdna4::lds_load16_nt(X + std::size_t{row} * attn::kDim + 16 * (pos ^ fp8_swz(r)),
                           lds + 1024 * i);
    }
  }
}

// The tile's 32 K then 32 V row scales (rows past last_row read last_row): 1 instruction.
__device__ __attribute__((always_inline)) inline void issue_fp8_scales(const float* KS,
                                                                      const float* VS,
                                                                      unsigned k0,
                                                                      unsigned last_row,
                                                                      unsigned lds,
                                                                      unsigned lane) {
  const unsigned r = k0 + (lane & 31u);
  const float* sw = ((lane & 32u) ? VS : KS) + (r <= last_row ? r : last_row);
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(sw), "s"(lds)
      : "memory");
}

typedef unsigned fp8_u32x2 __attribute__((ext_vector_type(2)));
typedef int fp8_i32x2 __attribute__((ext_vector_type(2)));

// Eight codes (bytes 0-7 of w) as an f16 x 8 operand, in byte order.
__device__ __attribute__((always_inline)) inline cdna4::half8_t widen8(unsigned w0, unsigned w1) {
  return __builtin_bit_cast(cdna4::half8_t,
                            cdna4::u32x4_t{fp8kv::pair_lo(w0), fp8kv::pair_hi(w0),
                                           fp8kv::pair_lo(w1), fp8kv::pair_hi(w1)});
}

// The raw operand codes of one stage. K: lane (g, c), key block kb, k-step s reads the 8 codes of
// dimensions 8 (4 s + g) .. + 7 of row 16 kb + c (chunk (2 s + g / 2) ^ c ^ 8 kb, half g % 2), at
// kaddr[kb] ^ 32 s, kaddr[kb] = K base + 4096 kb + 256 c + 32 (c / 2 ^ 4 kb) + 16 ((g / 2 ^ c) %
// 2) + 8 (g % 2). V^T: ds_read_b64_tr_b8 gives lane 16 G + 8 h + j byte j of the 8 bytes lanes
// 16 G + 2 k + h (k = 0 .. 7) supply, so lane 16 g + 2 k + h supplies dimensions 16 b + 8 h .. + 7
// of key 4 g + k (k < 4) or 16 + 4 g + k - 4, and lane (g, c) receives dimension 16 b + c of the
// keys of its k-slots 8 g .. 8 g + 7, in order: vaddr ^ 16 b, vaddr = V base + 256 key + 8 h + 16
// fp8_swz(key).
struct Fp8Raw {
  fp8_u32x2 k[2][8];
  fp8_i32x2 v[16];
};
__device__ __attribute__((always_inline)) inline void read_fp8_stage(Fp8Raw& raw,
                                                                    unsigned kaddr0,
                                                                    unsigned kaddr1,
                                                                    unsigned vaddr) {
#pragma unroll
  for (unsigned s = 0; s < 8; ++s)
#pragma unroll
    for (unsigned kb = 0; kb < 2; ++kb)
      raw.k[kb][s] = *reinterpret_cast<const __attribute__((address_space(3))) fp8_u32x2*>(
          (kb == 0 ? kaddr0 : kaddr1) ^ (32u * s));
#pragma unroll
  for (unsigned b = 0; b < 16; ++b)
    raw.v[b] = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
        reinterpret_cast<__attribute__((address_space(3))) fp8_i32x2*>(vaddr ^ (16u * b)));
}

// Partial (m, l, o) of keys [span.begin, span.end) of KV head kvh over e4m3 rows (K8 / V8 / KS /
// VS: the KV head's bases) at `base`, in the reference's partial layout (m: natural-log max of
// the scaled scores). `more`: the workgroup runs another item afterwards.
__device__ __attribute__((always_inline)) inline void split_partial_fp8_waves(
    const float* __restrict__ q, const uint8_t* K8, const uint8_t* V8, const float* KS,
    const float* VS, AttnSpan span, unsigned kvh, float* part_m, float* part_l, float* part_o,
    std::size_t base, Fp8WaveShared& sh, bool more) {
  using cdna4::half8_t;
  const unsigned t = threadIdx.x, lane = t & 63u, g = lane >> 4, c = lane & 15u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned n_tiles = (span.end - span.begin + kTileKeys - 1) / kTileKeys;
  const unsigned last_row = span.end - 1;  // unused when n_tiles == 0
  const unsigned nw = n_tiles > wave ? (n_tiles - wave + 3) / 4 : 0;
  unsigned off[2][4];
  fp8_copy_offsets(off, lane);
  // Tile j of the wave (ti = w + 4 j) into stage j % 2: K codes, scales, V codes (17
  // instructions).
  auto issue = [&](unsigned j) __attribute__((always_inline)) {
    const unsigned k0 = span.begin + (wave + 4 * j) * kTileKeys, st_ = j & 1u;
    const unsigned lds = cdna4::lds_offset(sh.codes[wave][st_]);
    issue_fp8_codes(K8, k0, last_row, lds, off, lane);
    issue_fp8_scales(KS, VS, k0, last_row, cdna4::lds_offset(sh.scale[wave][st_]), lane);
    issue_fp8_codes(V8, k0, last_row, lds + 8192u, off, lane);
  };

#pragma unroll
  for (unsigned i = 0; i < 2; ++i) {
    const unsigned h = 2 * wave + i;
    cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                      cdna4::lds_offset(sh.q[h]));
  }
  if (nw > 0)
    issue(0);
  if (nw > 1)
    issue(1);
  // The queries landed (the tiles' copies may be in flight).
  if (nw > 1)
    cdna4::wait_vmcnt<34>();
  else if (nw > 0)
    cdna4::wait_vmcnt<17>();
  else
    cdna4::wait_vmcnt<0>();
  tile_barrier();
  const TileLane tln = tile_lane(lane);
  WaveTileState st;
  wave_start(st, sh.q, lane, tln);
  const unsigned kl = 256 * c + 16 * (((g >> 1) ^ c) & 1u) + 8 * (g & 1u);
  const unsigned kl0 = kl + 32 * (c >> 1), kl1 = 4096 + kl + 32 * ((c >> 1) ^ 4u);
  unsigned vl;
  {
    const unsigned m = lane & 15u, k = m >> 1, h = m & 1u;
    const unsigned key = k < 4 ? 4 * g + k : 16 + 4 * g + (k - 4);
    vl = 8192 + 256 * key + 8 * h + 16 * fp8_swz(key);
  }
  float vref = 0.0f;  // R: the largest V row scale of the item's tiles so far (O is relative to it)

  // Tile j: in flight after its copies, those of tile j + 1 (17, if it exists). Every operand of
  // the tile is read into registers first; then tile j + 2 goes into its stage.
  for (unsigned j = 0; j < nw; ++j) {
    const unsigned ti = wave + 4 * j, st_ = j & 1u;
    if (j + 1 < nw)
      cdna4::wait_vmcnt<17>();
    else
      cdna4::wait_vmcnt<0>();
    const unsigned lds = cdna4::lds_offset(sh.codes[wave][st_]);
    Fp8Raw raw;
    read_fp8_stage(raw, lds + kl0, lds + kl1, lds + vl);
    const float* scl = sh.scale[wave][st_];
    const float4 ka4 = *reinterpret_cast<const float4*>(scl + 4 * g);
    const float4 kb4 = *reinterpret_cast<const float4*>(scl + 16 + 4 * g);
    const float4 va4 = *reinterpret_cast<const float4*>(scl + 32 + 4 * g);
    const float4 vb4 = *reinterpret_cast<const float4*>(scl + 48 + 4 * g);
    __builtin_amdgcn_sched_barrier(0);  // every read of the stage in flight
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (j + 2 < nw)
      issue(j + 2);
    // The lane's keys 4 g + i and 16 + 4 g + i (i < 4), in the order of its score values.
    const float ksc[8] = {ka4.x, ka4.y, ka4.z, ka4.w, kb4.x, kb4.y, kb4.z, kb4.w};
    const float vsc[8] = {va4.x, va4.y, va4.z, va4.w, vb4.x, vb4.y, vb4.z, vb4.w};
    half8_t ka[2][8];
#pragma unroll
    for (unsigned s = 0; s < 8; ++s)
#pragma unroll
      for (unsigned kb = 0; kb < 2; ++kb)
        ka[kb][s] = widen8(raw.k[kb][s].x, raw.k[kb][s].y);
    f32x4 s[2];
    wave_scores(s, ka, st);
    half8_t va[16];
#pragma unroll
    for (unsigned b = 0; b < 16; ++b)
      va[b] = widen8(static_cast<unsigned>(raw.v[b].x), static_cast<unsigned>(raw.v[b].y));
    // The tile's largest V row scale (rows past the span read the last row's): R moves up to it,
    // O by the exact power-of-two ratio (0 on the first tile, whose O is 0).
    const float vmax = cdna4::wave_allmax(
        fmaxf(fmaxf(fmaxf(vsc[0], vsc[1]), fmaxf(vsc[2], vsc[3])),
              fmaxf(fmaxf(vsc[4], vsc[5]), fmaxf(vsc[6], vsc[7]))));
    if (vmax > vref) {  // wave-uniform
      tile_scale_o(st.o, vref / vmax);
      vref = vmax;
    }
    const float inv = 1.0f / vref;  // a power of two: exact
    float vr[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vr[i] = vsc[i] * inv;
    const unsigned k0 = span.begin + ti * kTileKeys;
    TileSoftmax sm;
    if (k0 + kTileKeys > span.end)  // uniform
      tile_scores_joined<true, true>(sm, s, st.m, k0, span.end, lane, tln, ksc);
    else
      tile_scores_joined<false, true>(sm, s, st.m, k0, span.end, lane, tln, ksc);
    const bool first = j == 0;
    if (tile_decide<true>(sm, st, first, tln, vr))
      tile_rescale<true>(sm, st, first, tln, vr);
    st.l += sm.lt;
#pragma unroll
    for (int b2 = 0; b2 < 16; ++b2)
      st.o[b2] = mfma16(va[b2], sm.pb, st.o[b2]);
  }

  // The merge through stage 0 of each wave: wave w's result in its own (O in the first 8 KiB, mt
  // and l after it), which only it has used and which no copy still targets.
  {
    WaveResult r;
    wave_result(r, st, nw > 0, vref);
    float* mine = reinterpret_cast<float*>(sh.codes[wave][0]);
    wave_merge_store(mine, mine + 8 * attn::kDim, r, lane, 0, 16);
  }
  tile_barrier();
  {
    constexpr unsigned kStride = 2 * 16384 / 4;  // floats from one wave's stage 0 to the next
    const float* area = reinterpret_cast<const float*>(sh.codes[0][0]);
    const unsigned h = t % 8, d = t / 8;
    const WaveMergeScale ms = wave_merge_load_scale(area + 8 * attn::kDim, kStride, h);
    wave_merge_out(area, kStride, ms, d, d, h, part_o, base);
    wave_merge_out(area, kStride, ms, d + 32, d + 32, h, part_o, base);
    if (d == 0)
      wave_merge_ml_out(ms, h, part_m, part_l, base);
  }
  if (more)
    tile_barrier();  // LDS is reused by the next item
}

}  // namespace decode_detail

// Item = kvh * n_splits + split (grid-stride), launched as attn_split_kernel: dim3(n_splits, 2)
// x 256. Spans are attn_split_span's, so the partials line up with the f16 path's split for
// split, and attn_combine_kernel merges them.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_split_fp8_kernel(AttnSplitFp8Params p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::Fp8WaveShared sh;
  const unsigned count = attn::kKvHeads * p.n_splits;
  for (unsigned item = blockIdx.y * gridDim.x + blockIdx.x; item < count;
       item += gridDim.x * gridDim.y) {
    const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
    const std::size_t rows = std::size_t{kvh} * p.max_ctx;
    decode_detail::split_partial_fp8_waves(
        p.q, p.k8 + rows * attn::kDim, p.v8 + rows * attn::kDim, p.k_scale + rows,
        p.v_scale + rows, attn_split_span(p.len, p.n_splits, split), kvh, p.part_m, p.part_l,
        p.part_o, std::size_t{kvh} * p.n_splits + split, sh, item + gridDim.x * gridDim.y < count);
  }
}

}  // namespace miso::kernels
