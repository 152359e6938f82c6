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
//   attn_split_fp8_kernel<256>      split-K partials over e4m3 rows, in the reference's partial
//                                   layout; attn_combine_kernel merges them unchanged.

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

// An e4m3 unit is 16 rows: K rows at slot bytes [0, 4096), V rows at [4096, 8192), row r at
// 256 r -- the f16 unit's 8 KiB slot -- and 64 scales (K rows 0-15, V rows 0-15, then a copy).
constexpr unsigned kFp8UnitRows = 16;

constexpr int kFp8Ring = 2;  // units per wave's LDS ring: kFp8Ring - 1 in flight under one

template <int R>
struct SplitFp8SharedT {
  static constexpr int kWaveCount = kWaves, kRingUnits = R;
  SplitSharedT<kWaves, R> base;
  float scale[kWaves][R][64];
};
using SplitFp8Shared = SplitFp8SharedT<kFp8Ring>;

// Global -> LDS copy of one e4m3 unit: 4 row quads of K and of V (1 KiB each: row u0 + 4 i +
// lane / 16, bytes 16 (lane % 16)), then one 4-byte load per lane of the scales. `kw` / `vw` are
// the lane's addresses in quad 0, `sw` its scale address. 9 vector-memory instructions.
__device__ __attribute__((always_inline)) inline void issue_unit_fp8(const uint8_t* kw,
                                                                     const uint8_t* vw,
                                                                     const float* sw,
                                                                     unsigned slot_lds,
                                                                     unsigned scale_lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %4\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:3072 nt\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:3072 nt\n\t"
      "s_mov_b32 m0, %6\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %3, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(kw), "v"(vw), "v"(sw), "s"(slot_lds), "s"(slot_lds + 4096u), "s"(scale_lds)
      : "memory");
}

// The same copy for the unit that crosses the end of the cache: rows past last_row are clamped
// to it (they are masked at use). K8 / V8 / KS / VS are the KV head's bases. Also 9 instructions.
__device__ __attribute__((always_inline)) inline void issue_unit_fp8_clamped(
    const uint8_t* K8, const uint8_t* V8, const float* KS, const float* VS, unsigned u0,
    unsigned last_row, unsigned slot_lds, unsigned scale_lds, unsigned lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned row = u0 + 4 * i + (lane >> 4);
    row = row < last_row ? row : last_row;
    const std::size_t at = std::size_t{row} * attn::kDim + (lane & 15u) * 16;
    cdna4::lds_load16_nt(K8 + at, slot_lds + 1024 * i);
    cdna4::lds_load16_nt(V8 + at, slot_lds + 4096 + 1024 * i);
  }
  unsigned row = u0 + (lane & 15u);
  row = row < last_row ? row : last_row;
  const float* sw = ((lane & 16u) ? VS : KS) + row;
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(sw), "s"(scale_lds)
      : "memory");
}

// Wait until the unit whose copy was followed by `after` (< 4) more units' copies has landed.
__device__ __attribute__((always_inline)) inline void wait_fp8_units_after(unsigned after) {
  switch (after) {
    case 0: cdna4::wait_vmcnt<0>(); break;
    case 1: cdna4::wait_vmcnt<9>(); break;
    case 2: cdna4::wait_vmcnt<18>(); break;
    default: cdna4::wait_vmcnt<27>(); break;
  }
}

// One 8-row half of an e4m3 unit: the lane layout of process_unit, with the K chunk of a row
// being dimensions 16 dc .. 16 dc + 15 (16 bytes) and the V chunk dimensions 8 c .. 8 c + 7 of
// rows 2 i + a (8 bytes). Codes widen to f16 exactly; the row scales enter through
// unit_numerators: scores x K scale (f32), numerators x the row's V scale relative to the unit's
// largest (vratio <= 1, so the f16 numerator never exceeds the unscaled one). The half's P V
// accumulates into the unit's f32 sums t (kFirst: the unit's first half starts them).
template <bool kFirst>
__device__ __attribute__((always_inline)) inline void process_half_fp8(
    WaveState& st, const uint4 (&kr)[4], const uint2 (&vr)[4], float ksc, float vratio,
    const half2_t (&qh)[4][8], unsigned r0, unsigned span_end, uint32_t (*pbuf)[2][kGroup],
    float (&t)[kGroup][8], unsigned lane) {
  float part[16];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const unsigned w[4] = {kr[rr].x, kr[rr].y, kr[rr].z, kr[rr].w};
    unsigned kh[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kh[2 * i] = fp8kv::pair_lo(w[i]);
      kh[2 * i + 1] = fp8kv::pair_hi(w[i]);
    }
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float acc = dot2_first(qh[hh][0], kh[0]);
#pragma unroll
      for (int j = 1; j < 8; ++j)
        acc = __builtin_amdgcn_fdot2(qh[hh][j], cdna4::as_half2(kh[j]), acc, false);
      part[4 * hh + rr] = acc;
    }
  }
  const float m_before = st.m;
  unit_numerators<true>(st, part, r0, span_end, ksc, vratio, pbuf, lane);
  if constexpr (!kFirst) {
    // The first half's sums in t were taken against the previous reference max: when this
    // half moved it, t takes the same per-head correction as o (unit_softmax_state's).
    if (__builtin_amdgcn_ballot_w64(st.m != m_before)) {  // wave-uniform branch
      const float corr = __builtin_amdgcn_exp2f(m_before - st.m);
#pragma unroll
      for (int h = 0; h < kGroup; ++h) {
        const float ch =
            cdna4::as_float(__builtin_amdgcn_readlane(cdna4::as_uint(corr), head_lane(h)));
#pragma unroll
        for (int e = 0; e < 8; ++e)
          t[h][e] *= ch;
      }
    }
  }
  // P V over this lane's rows 2 i + a, dimensions 8 c .. 8 c + 7: the byte permutes interleave
  // rows 2 g + a and 2 g + 4 + a so that one conversion yields their f16 pair for a dimension.
  const unsigned a = lane >> 5;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint4 p0 = *reinterpret_cast<const uint4*>(&pbuf[a][g][0]);
    const uint4 p1 = *reinterpret_cast<const uint4*>(&pbuf[a][g][4]);
    const unsigned pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    const unsigned r0w[2] = {vr[g].x, vr[g].y}, r1w[2] = {vr[g + 2].x, vr[g + 2].y};
    unsigned pv[8];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const unsigned lo = __builtin_amdgcn_perm(r1w[j], r0w[j], 0x05010400u);
      const unsigned hi = __builtin_amdgcn_perm(r1w[j], r0w[j], 0x07030602u);
      pv[4 * j + 0] = fp8kv::pair_lo(lo);
      pv[4 * j + 1] = fp8kv::pair_hi(lo);
      pv[4 * j + 2] = fp8kv::pair_lo(hi);
      pv[4 * j + 3] = fp8kv::pair_hi(hi);
    }
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (kFirst && g == 0)
          t[h][e] = dot2_first(cdna4::as_half2(pp[h]), pv[e]);
        else
          t[h][e] = __builtin_amdgcn_fdot2(cdna4::as_half2(pp[h]), cdna4::as_half2(pv[e]),
                                           t[h][e], false);
      }
  }
}

// One 16-row e4m3 unit: every LDS read of both halves first, then the halves in order. The
// unit's V reference is its largest V row scale among the rows of the span (wave-uniform): the
// numerators carry each row's scale relative to it, the unit's P V sums stay in f32 and enter o
// times the reference. A common power-of-two factor on every V scale therefore leaves the f16
// numerators unchanged (no f16 overflow at the largest scales, no underflow at the smallest);
// only the spread of V scales within 16 consecutive rows scales them down.
__device__ __attribute__((always_inline)) inline void process_unit_fp8(
    WaveState& st, const unsigned char* slot, const float* scl, const unsigned (&koff)[4],
    const half2_t (&qh)[4][8], unsigned u0, unsigned span_end, uint32_t (*pbuf)[2][kGroup],
    unsigned lane) {
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, a = lane >> 5, c = lane & 31u;
  const unsigned srow = 4 * rq + (dc & 3u);  // the lane's score row within a half
  uint4 kr[2][4];
  uint2 vr[2][4];
  float ksc[2], vsc[2];
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      kr[hf][rr] = *reinterpret_cast<const uint4*>(slot + 2048 * hf + koff[rr]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      vr[hf][i] = *reinterpret_cast<const uint2*>(slot + 4096 + 2048 * hf + 512 * i + 256 * a +
                                                  8 * c);
    ksc[hf] = scl[8 * hf + srow];
    vsc[hf] = scl[16 + 8 * hf + srow];
  }
  __builtin_amdgcn_sched_barrier(0);
  // Rows past the span are masked (p = 0) and stay out of the reference; row u0 is in the span.
  const float v0 = u0 + srow < span_end ? vsc[0] : 0.0f;
  const float v1 = u0 + 8 + srow < span_end ? vsc[1] : 0.0f;
  const float uref = cdna4::wave_allmax(fmaxf(v0, v1));
  const float inv = uref > 0.0f ? 1.0f / uref : 0.0f;
  float t[kGroup][8];
  process_half_fp8<true>(st, kr[0], vr[0], ksc[0], vsc[0] * inv, qh, u0, span_end, pbuf, t,
                         lane);
  process_half_fp8<false>(st, kr[1], vr[1], ksc[1], vsc[1] * inv, qh, u0 + 8, span_end, pbuf, t,
                          lane);
#pragma unroll
  for (int h = 0; h < kGroup; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      st.o[h][e] = __builtin_fmaf(t[h][e], uref, st.o[h][e]);
}

// Partial (m, l, o) of keys [span.begin, span.end) for KV head kvh over e4m3 rows (K8 / V8 /
// KS / VS: the KV head's bases), written at `base` in the reference's partial layout. The same
// schedule as split_partial_rows with 16-row units: wave w streams units starting at rows
// span.begin + 16 w, + 64, ... through its kRingUnits-unit LDS ring; rows past the span are
// masked and rows past len - 1 are never read.
template <class Shared>
__device__ __attribute__((always_inline)) inline void split_partial_fp8(
    const float* __restrict__ q, const uint8_t* K8, const uint8_t* V8, const float* KS,
    const float* VS, unsigned len, AttnSpan span, unsigned kvh, float* part_m, float* part_l,
    float* part_o, std::size_t base, Shared& sh, bool more) {
  constexpr int kW = Shared::kWaveCount, kR = Shared::kRingUnits;
  static_assert(kR >= 2 && kR <= 4 && kW == kWaves, "ring depth / wave count");
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned last_row = len - 1;
  constexpr unsigned kStride = kW * kFp8UnitRows;
  const unsigned first = span.begin + wave * kFp8UnitRows;
  const unsigned n_units = first < span.end ? (span.end - first + kStride - 1) / kStride : 0;
  const unsigned ring0 = cdna4::lds_offset(sh.base.ring[wave][0]);
  const unsigned scale0 = cdna4::lds_offset(sh.scale[wave][0]);
  // This lane's bytes of row quad 0 of unit 0 and its scale (K rows for lanes 0-15 of each
  // half-wave, V rows for 16-31); unit k is kStride rows further.
  const std::size_t lane_at = std::size_t{first + (lane >> 4)} * attn::kDim + (lane & 15u) * 16;
  const float* lane_scale = ((lane & 16u) ? VS : KS) + first + (lane & 15u);
  auto issue = [&](unsigned k) {
    const unsigned u0 = first + k * kStride;
    const unsigned slot = ring0 + (k % kR) * kUnitBytes;
    const unsigned sslot = scale0 + (k % kR) * 256;
    if (u0 + kFp8UnitRows <= len) {  // wave-uniform
      const std::size_t step = std::size_t{k} * kStride * attn::kDim;
      issue_unit_fp8(K8 + lane_at + step, V8 + lane_at + step, lane_scale + k * kStride, slot,
                     sslot);
    } else {
      issue_unit_fp8_clamped(K8, V8, KS, VS, u0, last_row, slot, sslot, lane);
    }
  };

  // This wave's query heads of the KV head (1 KiB each), then the first kR - 1 units.
  constexpr int kHeadsPerWave = kGroup / kW;
#pragma unroll
  for (int i = 0; i < kHeadsPerWave; ++i) {
    const unsigned h = kHeadsPerWave * wave + i;
    cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                      cdna4::lds_offset(sh.base.q[h]));
  }
#pragma unroll
  for (unsigned k = 0; k + 1 < kR; ++k)
    if (k < n_units)
      issue(k);
  wait_fp8_units_after(n_units < kR - 1 ? n_units : kR - 1);  // the query loads are older
  __syncthreads();

  // Query slices as f16 pairs pre-scaled by log2(e)/16: slot hh = head 4 hq + (hh ^ dc / 4),
  // pair j = dimensions 16 dc + 2 j, 16 dc + 2 j + 1.
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, hq = lane >> 5;
  half2_t qh[4][8];
  constexpr float kScale = kLog2e / 16.0f;  // 1/sqrt(256) in log2 units
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    const unsigned h = 4 * hq + (hh ^ (dc >> 2));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 x = *reinterpret_cast<const float4*>(&sh.base.q[h][16 * dc + 4 * i]);
      qh[hh][2 * i] = half2_t{static_cast<_Float16>(x.x * kScale),
                              static_cast<_Float16>(x.y * kScale)};
      qh[hh][2 * i + 1] = half2_t{static_cast<_Float16>(x.z * kScale),
                                  static_cast<_Float16>(x.w * kScale)};
    }
  }
  // K read offsets in a half: row 4 rq + (rr ^ dc % 4), 16-byte chunk dc.
  unsigned koff[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    koff[rr] = (4 * rq + (rr ^ (dc & 3u))) * 256 + 16 * dc;

  WaveState st;
  st.m = -__builtin_inff();
  st.mt = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int h = 0; h < kGroup; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      st.o[h][e] = 0.0f;

  unsigned k = 0;
  for (; k + kR - 1 < n_units; ++k) {
    issue(k + kR - 1);
    cdna4::wait_vmcnt<9 * (kR - 1)>();
    process_unit_fp8(st, sh.base.ring[wave][k % kR], sh.scale[wave][k % kR], koff, qh,
                     first + k * kStride, span.end, sh.base.p[wave], lane);
  }
  for (; k < n_units; ++k) {
    wait_fp8_units_after(n_units - 1 - k);
    process_unit_fp8(st, sh.base.ring[wave][k % kR], sh.scale[wave][k % kR], koff, qh,
                     first + k * kStride, span.end, sh.base.p[wave], lane);
  }
  write_partial(st, sh.base, part_m, part_l, part_o, base, more);
}

}  // namespace decode_detail

// Item = kvh * n_splits + split (grid-stride), launched as attn_split_kernel: dim3(n_splits, 2)
// x 256. Spans are attn_split_span's, so the partials line up with the f16 path's split for
// split, and attn_combine_kernel merges them.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_split_fp8_kernel(AttnSplitFp8Params p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::SplitFp8Shared sh;
  const unsigned count = attn::kKvHeads * p.n_splits;
  for (unsigned item = blockIdx.y * gridDim.x + blockIdx.x; item < count;
       item += gridDim.x * gridDim.y) {
    const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
    const std::size_t rows = std::size_t{kvh} * p.max_ctx;
    decode_detail::split_partial_fp8(
        p.q, p.k8 + rows * attn::kDim, p.v8 + rows * attn::kDim, p.k_scale + rows,
        p.v_scale + rows, p.len, attn_split_span(p.len, p.n_splits, split), kvh, p.part_m,
        p.part_l, p.part_o, std::size_t{kvh} * p.n_splits + split, sh,
        item + gridDim.x * gridDim.y < count);
  }
}

}  // namespace miso::kernels
