#pragma once

// Gated GQA softmax attention, decode path, for MI355X (gfx950 / CDNA4).
//
// Shapes (qwen3_5_moe full-attention layer): 16 query heads, 2 KV heads (GQA 8:1), head_dim 256,
// partial NEOX RoPE on the first 64 dims, f16 KV cache laid out [kv_head][max_ctx][256].
//
// Source-compatible drop-in for miso's kernels/attention_decode.hpp: the Params structs keep the
// reference's field order and types (callers use positional aggregate init), and the kernel and
// helper templates keep their names and template parameters, so src/engine/attention.hip,
// tests/test_attn_splitk.hip and bench/attention compile unchanged against this header. The kernel
// bodies are new: see the comment above each op.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "cdna4_wave.hpp"

namespace miso::kernels {

namespace attn {
constexpr int kQHeads = 16, kKvHeads = 2, kDim = 256, kRopeDim = 64;
typedef _Float16 half_t;
}  // namespace attn

// ------------------------------------------------------------------------------------------------
// Prep: per-head RMSNorm + NEOX RoPE + f16 KV append (reference: kernels/attention_decode.hpp:19-83)
// ------------------------------------------------------------------------------------------------

struct AttnPrepParams {
  const float* qg;        // [16][512]: per head 256 query then 256 gate (q projection output)
  const float* k;         // [2][256]
  const float* v;         // [2][256]
  const float* q_norm;    // [256], GGUF stores 1 + w
  const float* k_norm;    // [256]
  const float* inv_freq;  // [32]
  attn::half_t* k_cache;  // [2][max_ctx][256]
  attn::half_t* v_cache;  // [2][max_ctx][256]
  float* q;               // [16][256] normalised, rotated queries
  unsigned pos, max_ctx;
  float eps;
};

// Prefill form: token t reads qg/k/v at t * proj_stride floats past tok0's pointers, writes q at
// t * 4096 floats and the cache at position pos + t.
struct AttnPrepBatchParams {
  AttnPrepParams tok0;
  unsigned n;
  unsigned proj_stride;
};

namespace decode_detail {

// Thread d's value of head `head` of 18 (0..15 query heads, 16..17 KV heads) after RMSNorm and
// NEOX RoPE, on a 256-thread workgroup, thread d owning dimension d. The sum of squares is a
// wave64 butterfly plus a 4-entry LDS exchange (wave_ss, free again on return); the RoPE partner
// (d +- 32) is lane ^ 32 of wave 0, read through the lane crossbar, so no LDS staging. P is any
// params struct with the qg / k / q_norm / k_norm / inv_freq / pos / eps fields of
// AttnPrepParams.
template <int kBlock, class P>
__device__ __attribute__((always_inline)) inline float prep_value(const P& p, unsigned head,
                                                                  float* wave_ss) {
  using namespace attn;
  static_assert(kBlock == kDim, "one thread per dimension");
  const unsigned d = threadIdx.x;
  const bool is_q = head < static_cast<unsigned>(kQHeads);
  const unsigned kvh = head - kQHeads;
  float x = is_q ? p.qg[head * 2 * kDim + d] : p.k[kvh * kDim + d];
  const float ss_wave = cdna4::wave_allsum(x * x);
  if ((d & 63u) == 0)
    wave_ss[d >> 6] = ss_wave;
  __syncthreads();
  const float ss = (wave_ss[0] + wave_ss[1]) + (wave_ss[2] + wave_ss[3]);
  __syncthreads();  // wave_ss is reused by the next head of a grid-stride loop
  const float r = rsqrtf(ss / kDim + p.eps);
  x = x * r * (is_q ? p.q_norm[d] : p.k_norm[d]);
  if (d < static_cast<unsigned>(kRopeDim)) {  // wave 0 only: uniform for the crossbar read
    constexpr unsigned kHalf = kRopeDim / 2;
    const float partner = cdna4::lane_xor32(x);
    float s, c;
    sincosf(static_cast<float>(p.pos) * p.inv_freq[d % kHalf], &s, &c);
    x = d < kHalf ? x * c - partner * s : x * c + partner * s;
  }
  return x;
}

}  // namespace decode_detail

// One head of 18 on a 256-thread workgroup (prep_value), then the store: the query row, or the
// f16 K and V rows at position pos.
template <int kBlock>
__device__ void attn_prep_head(const AttnPrepParams& p, unsigned head) {
  using namespace attn;
  __shared__ float wave_ss[kBlock / cdna4::kLanes];
  const unsigned d = threadIdx.x;
  const float x = decode_detail::prep_value<kBlock>(p, head, wave_ss);
  if (head < static_cast<unsigned>(kQHeads)) {
    p.q[head * kDim + d] = x;
  } else {
    const unsigned kvh = head - kQHeads;
    const std::size_t at = (std::size_t{kvh} * p.max_ctx + p.pos) * kDim + d;
    p.k_cache[at] = static_cast<half_t>(x);
    p.v_cache[at] = static_cast<half_t>(p.v[kvh * kDim + d]);
  }
}

// Heads [first, first + count) of 18, one workgroup per head (grid-stride).
template <int kBlock>
__device__ void attn_prep_op(const AttnPrepParams& p, unsigned first, unsigned count) {
  for (unsigned head = first + blockIdx.x; head < first + count; head += gridDim.x)
    attn_prep_head<kBlock>(p, head);
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prep_kernel(AttnPrepParams p) {
  attn_prep_op<kBlock>(p, 0, attn::kQHeads + attn::kKvHeads);
}

// ------------------------------------------------------------------------------------------------
// Split-K decode (reference: kernels/attention_decode.hpp:85-236)
// ------------------------------------------------------------------------------------------------

// Header constant kept for source compatibility; the MI355X kernels walk keys in units of
// kAttnDecodeUnit rows per wave.
constexpr unsigned kAttnSubChunk = 32;
constexpr unsigned kAttnDecodeUnit = 8;

// Split-count policy for MI355X: one split per 32 keys (short contexts stay latency-bound, so more
// workgroups help), at most 128 splits per KV head (2 x 128 workgroups fill 256 CUs once), never
// more than the caller's partial-buffer capacity max_splits. len = 0 -> 1. Always 1 <= n <=
// max(max_splits, 1).
constexpr unsigned kAttnTargetSplits = 128;
__host__ __device__ constexpr unsigned attn_n_splits(unsigned len, unsigned max_splits) {
  const unsigned want = (len + kAttnSubChunk - 1) / kAttnSubChunk;
  unsigned cap = max_splits < kAttnTargetSplits ? max_splits : kAttnTargetSplits;
  if (cap == 0)
    cap = 1;
  const unsigned n = want < cap ? want : cap;
  return n == 0 ? 1 : n;
}

// Key span [begin, end) of one split: whole kAttnDecodeUnit-row units, split i taking units
// [i * per, (i + 1) * per) with per = ceil(units / n_splits). Trailing splits may be empty.
struct AttnSpan {
  unsigned begin, end;
};
__host__ __device__ inline AttnSpan attn_split_span(unsigned len, unsigned n_splits,
                                                    unsigned split) {
  const unsigned units = (len + kAttnDecodeUnit - 1) / kAttnDecodeUnit;
  const unsigned per = (units + n_splits - 1) / n_splits;
  const unsigned long long b = 1ull * split * per * kAttnDecodeUnit;
  const unsigned begin = b < len ? static_cast<unsigned>(b) : len;
  const unsigned long long e = b + 1ull * per * kAttnDecodeUnit;
  return {begin, e < len ? static_cast<unsigned>(e) : len};
}

struct AttnSplitParams {
  const float* q;               // [16][256] (unscaled)
  const attn::half_t* k_cache;  // [2][max_ctx][256]
  const attn::half_t* v_cache;
  float* part_m;  // [2][n_splits][8] running max of scaled scores (natural log units)
  float* part_l;  // [2][n_splits][8] sum of exp(score - max)
  float* part_o;  // [2][n_splits][8][256] sum of exp(score - max) V
  unsigned len, max_ctx, n_splits;
};

namespace decode_detail {

using cdna4::half2_t;
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.693147180559945309417f;
constexpr int kGroup = attn::kQHeads / attn::kKvHeads;  // 8 query heads per KV head
constexpr int kWaves = 4;                               // 256-thread workgroup (header API)

constexpr int kRing = 2;               // units per wave in the LDS ring: one loads under one
constexpr unsigned kUnitBytes = 8192;  // 8 K rows (4 KiB) then 8 V rows (4 KiB), natural order
constexpr float kRescaleSlack = 8.0f;  // log2 units: numerators stay <= 2^8 between rescales

// LDS of one split workgroup: each wave's ring of K/V units (direct global->LDS loads), the query
// rows, per-wave softmax numerators (f16 pairs) and per-wave head statistics; the cross-wave
// merge of the value accumulators reuses the ring.
template <int W, int R>
struct SplitSharedT {
  static constexpr int kWaveCount = W, kRingUnits = R;
  // Each wave's ring of units; after its stream, slot 0 of a wave's ring holds that wave's
  // value accumulators for the cross-wave merge ([head][dim], 8 x 256 floats = 8 KiB), so a
  // wave that finishes early never writes into a ring another wave still streams through.
  unsigned char ring[W][R][kUnitBytes];
  float q[kGroup][attn::kDim];
  // Numerators of one unit as f16 pairs, [wave][row parity a][pair g][head]: the pair holds rows
  // 2 g + a and 2 g + 4 + a of the unit (f16-query arithmetic).
  uint32_t p[W][2][2][kGroup];
  // Numerators of one unit in f32, [wave][unit row][head] (f32 arithmetic).
  float pf[W][kAttnDecodeUnit][kGroup];
  float stat_m[W][kGroup], stat_mt[W][kGroup], stat_l[W][2][kGroup];
  static_assert(sizeof(float) * kGroup * attn::kDim <= kUnitBytes,
                "a wave's merge rows must fit in one slot of its own ring");
  __device__ float* merge_rows(int w) { return reinterpret_cast<float*>(ring[w][0]); }
};
using SplitShared = SplitSharedT<kWaves, kRing>;

// Global -> LDS copy of one unit: K rows u0 .. u0 + 7 to slot bytes [0, 4096), V rows to [4096,
// 8192), row r at 512 r. One instruction moves one row pair (1 KiB, 16 bytes per lane); `kw` / `vw`
// are this lane's addresses of the first pair (row u0 + lane / 32, bytes 16 (lane % 32) of it).
// The instruction offset advances the global and the LDS address together, which is exactly the
// 1 KiB step of both layouts, so one address register serves all four pairs. The loads carry the
// non-temporal hint: the cache is streamed once per call. M0 is saved and restored.
__device__ __attribute__((always_inline)) inline void issue_unit(const attn::half_t* kw,
                                                                 const attn::half_t* vw,
                                                                 unsigned slot_lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %1, off offset:3072 nt\n\t"
      "s_mov_b32 m0, %4\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, off nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %2, off offset:3072 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(kw), "v"(vw), "s"(slot_lds), "s"(slot_lds + 4096u)
      : "memory");
}

// The same copy for the unit that crosses the end of the cache (len): rows past len - 1 are
// clamped to it (they are masked at use), so no load leaves [0, len). Also 8 instructions.
__device__ __attribute__((always_inline)) inline void issue_unit_clamped(
    const attn::half_t* K, const attn::half_t* V, unsigned u0, unsigned last_row,
    unsigned slot_lds, unsigned lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned row = u0 + 2 * i + (lane >> 5);
    row = row < last_row ? row : last_row;
    const std::size_t at = std::size_t{row} * attn::kDim + (lane & 31u) * 8;
    cdna4::lds_load16_nt(K + at, slot_lds + 1024 * i);
    cdna4::lds_load16_nt(V + at, slot_lds + 4096 + 1024 * i);
  }
}

// Wait until the unit whose copy was followed by `after` (< 4) more units' copies has landed
// (8 vector-memory instructions per unit).
__device__ __attribute__((always_inline)) inline void wait_units_after(unsigned after) {
  switch (after) {
    case 0: cdna4::wait_vmcnt<0>(); break;
    case 1: cdna4::wait_vmcnt<8>(); break;
    case 2: cdna4::wait_vmcnt<16>(); break;
    default: cdna4::wait_vmcnt<24>(); break;
  }
}

// Running state of one wave.
//   Scores: lane = (hq = lane / 32, rq = lane / 16 % 2, dc = lane % 16) owns head 4 hq + dc / 4
//   and unit row 4 rq + dc % 4 after the reduction; m (reference max), mt (true max), both log2
//   units and uniform over the head's 8 lanes, and l (this lane's share of the head's sum) follow
//   that head.
//   Values: lane = (a = lane / 32, c = lane % 32) accumulates o[h][e] = head h, dimension 8 c + e,
//   over the unit rows of parity a, relative to m.
struct WaveState {
  float m, mt, l;
  float o[kGroup][8];
};

// Lane holding head h's statistics (rq = 0, dc = 4 (h % 4)).
__device__ inline unsigned head_lane(int h) { return 32u * (h >> 2) + 4u * (h & 3); }

// v_dot2_f32_f16 with a zero accumulator (the VOP3 form takes the inline constant, so no register
// has to be cleared first).
__device__ __attribute__((always_inline)) inline float dot2_first(half2_t a, unsigned b) {
  float r;
  asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// The part of one unit's online softmax that does not depend on the cache format: the
// reduce-scatter of the lane's 16 partial dot products (see process_unit) to one score per lane
// (head 4 hq + dc / 4, unit row 4 rq + dc % 4), the span mask, the lazy rescale, and the f16
// numerators, published to `pbuf` for P V. With kScaled, the score is multiplied by its row's K
// scale and the published numerator by vsc, the row's V scale relative to its unit's largest
// (vsc <= 1; the l sum stays unscaled).
// The reduce-scatter of the lane's 16 partial dot products (see process_unit) over the 16 lanes
// of dc: returns the complete score of head 4 hq + dc / 4, unit row 4 rq + dc % 4.
__device__ __attribute__((always_inline)) inline float unit_scores(const float (&part)[16]) {
  float r8[8], r4[4], r2[2];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    r8[j] = part[j] + cdna4::dpp_mov<cdna4::kRowRor8>(part[j ^ 8]);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    r4[j] = r8[j] + cdna4::dpp_mov<cdna4::kRowHalfMirror>(r8[j ^ 7]);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    r2[j] = r4[j] + cdna4::dpp_mov<cdna4::kQuadXor2>(r4[j ^ 2]);
  return r2[0] + cdna4::dpp_mov<cdna4::kQuadXor1>(r2[1]);
}

// Span mask, head max and lazy rescale of one unit's scores (lane layout of unit_scores): masks
// rows past span_end to -inf, raises the true max mt, and moves the reference max m (rescaling l
// and the value accumulators) only when the unit's head max exceeds it by more than the slack.
// Returns the lane's (masked) score.
__device__ __attribute__((always_inline)) inline float unit_softmax_state(WaveState& st, float s,
                                                                          unsigned u0,
                                                                          unsigned span_end,
                                                                          unsigned lane) {
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u;
  const unsigned row = 4 * rq + (dc & 3u);
  if (u0 + row >= span_end)
    s = -__builtin_inff();
  // Head max over its 8 lanes (dc % 4 and rq). Row u0 is always in the span, so every head has
  // a finite score.
  float mu = fmaxf(s, cdna4::dpp_mov<cdna4::kQuadXor1>(s));
  mu = fmaxf(mu, cdna4::dpp_mov<cdna4::kQuadXor2>(mu));
  mu = cdna4::max_xor16(mu);
  st.mt = fmaxf(st.mt, mu);
  if (__builtin_amdgcn_ballot_w64(mu > st.m + kRescaleSlack)) {  // wave-uniform branch
    const float m_new = fmaxf(st.m, mu);
    const float corr = __builtin_amdgcn_exp2f(st.m - m_new);  // 0 on the first unit (m = -inf)
    st.l *= corr;
    st.m = m_new;
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
      const float ch =
          cdna4::as_float(__builtin_amdgcn_readlane(cdna4::as_uint(corr), head_lane(h)));
#pragma unroll
      for (int e = 0; e < 8; ++e)
        st.o[h][e] *= ch;
    }
  }
  return s;
}

template <bool kScaled>
__device__ __attribute__((always_inline)) inline void unit_numerators(
    WaveState& st, const float (&part)[16], unsigned u0, unsigned span_end, float ksc, float vsc,
    uint32_t (*pbuf)[2][kGroup], unsigned lane) {
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, hq = lane >> 5;
  float s = unit_scores(part);
  if constexpr (kScaled)
    s *= ksc;
  const unsigned row = 4 * rq + (dc & 3u);
  s = unit_softmax_state(st, s, u0, span_end, lane);
  const _Float16 p16 = static_cast<_Float16>(__builtin_amdgcn_exp2f(s - st.m));  // 0 if masked
  st.l += static_cast<float>(p16);  // the sum of exactly the numerators P V uses
  {
    const unsigned head = 4 * hq + (dc >> 2);
    _Float16* ph = reinterpret_cast<_Float16*>(&pbuf[row & 1u][(row >> 1) & 1u][head]);
    if constexpr (kScaled)
      ph[row >> 2] = static_cast<_Float16>(static_cast<float>(p16) * vsc);
    else
      ph[row >> 2] = p16;
  }
}

// One unit (8 rows) of the online softmax.
//
// S: the lane's 16 partial dot products (4 heads x 4 rows, 16 of its dimensions each) are laid
// out so that a reduce-scatter over the 16 lanes of dc needs one DPP add per value and level:
// register slot s = 4 hh + rr holds head 4 hq + (hh ^ dc / 4) and row 4 rq + (rr ^ dc % 4), i.e.
// value index s ^ dc. At a level with lane mask mu (8, 7, 2, 1: highest bits 3..0) every lane
// keeps slots j < mu's top bit and adds the partner's slot j ^ mu, which holds the same value
// index; after four levels lane dc holds value dc. The query slots hh are permuted per lane once
// at the start; the row permutation is folded into the lane's LDS read addresses.
// P V: rows (2 g + a, 2 g + 4 + a) pair up in one v_dot2_f32_f16 per (head, dimension); their
// numerators arrive as f16 pairs through a 128-byte per-wave LDS buffer.
__device__ __attribute__((always_inline)) inline void process_unit(
    WaveState& st, const unsigned char* slot, const unsigned (&koff)[4],
    const half2_t (&qh)[4][8], unsigned u0, unsigned span_end, uint32_t (*pbuf)[2][kGroup],
    unsigned lane) {
  // All of the unit's K and V reads first, so their LDS latency overlaps.
  uint4 kr[4][2], vr[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    kr[rr][0] = *reinterpret_cast<const uint4*>(slot + koff[rr]);
    kr[rr][1] = *reinterpret_cast<const uint4*>(slot + koff[rr] + 256);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    vr[i] = *reinterpret_cast<const uint4*>(slot + 4096 + 1024 * i + 16 * lane);
  __builtin_amdgcn_sched_barrier(0);
  float part[16];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const uint4 k0 = kr[rr][0], k1 = kr[rr][1];
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float acc = dot2_first(qh[hh][0], k0.x);
      acc = __builtin_amdgcn_fdot2(qh[hh][1], cdna4::as_half2(k0.y), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][2], cdna4::as_half2(k0.z), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][3], cdna4::as_half2(k0.w), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][4], cdna4::as_half2(k1.x), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][5], cdna4::as_half2(k1.y), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][6], cdna4::as_half2(k1.z), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[hh][7], cdna4::as_half2(k1.w), acc, false);
      part[4 * hh + rr] = acc;
    }
  }
  unit_numerators<false>(st, part, u0, span_end, 1.0f, 1.0f, pbuf, lane);
  // P V over this lane's rows 2 i + a, dimensions 8 c .. 8 c + 7.
  const unsigned a = lane >> 5;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint4 p0 = *reinterpret_cast<const uint4*>(&pbuf[a][g][0]);
    const uint4 p1 = *reinterpret_cast<const uint4*>(&pbuf[a][g][4]);
    const unsigned pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    const unsigned r0[4] = {vr[g].x, vr[g].y, vr[g].z, vr[g].w};
    const unsigned r1[4] = {vr[g + 2].x, vr[g + 2].y, vr[g + 2].z, vr[g + 2].w};
    half2_t pv[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pv[2 * j] = cdna4::as_half2(__builtin_amdgcn_perm(r1[j], r0[j], 0x05040100u));
      pv[2 * j + 1] = cdna4::as_half2(__builtin_amdgcn_perm(r1[j], r0[j], 0x07060302u));
    }
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        st.o[h][e] = __builtin_amdgcn_fdot2(cdna4::as_half2(pp[h]), pv[e], st.o[h][e], false);
  }
}

// The arithmetic of a split: the reference's (kernels/attention_decode.hpp:150-221: an f32
// query, f32 scores, f32 numerators, f32 P V over f16 K/V widened exactly) or an f16 query and
// f16 numerators through v_dot2_f32_f16 (two products per instruction, per-head rel-L2 ~3e-4).
enum class DecodeArith { kF32, kF16Query };

// One unit (8 rows) of the online softmax in f32 arithmetic. The lane layout is process_unit's;
// every product is one v_fma_mix_f32 (an f16 operand widened exactly, f32 fused multiply-add).
// S: the lane's 16 partial dot products (4 heads x 4 rows over its 16 dimensions) from its f32
// query slice `qf` (slot hh = head 4 hq + (hh ^ dc / 4); entries 0-7 = dimensions 8 dc + j,
// 8-15 = 128 + 8 dc + j) -- 256 products per lane. P V: o[h][e] over the lane's rows 2 i + a and
// dimensions 8 c + e with the unit's f32 numerators from the per-wave buffer `pf[row][head]` --
// another 256.
__device__ __attribute__((always_inline)) inline void process_unit_f32(
    WaveState& st, const unsigned char* slot, const unsigned (&koff)[4], const float (&qf)[4][16],
    unsigned u0, unsigned span_end, float (*pf)[kGroup], unsigned lane) {
  uint4 kr[4][2], vr[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    kr[rr][0] = *reinterpret_cast<const uint4*>(slot + koff[rr]);
    kr[rr][1] = *reinterpret_cast<const uint4*>(slot + koff[rr] + 256);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    vr[i] = *reinterpret_cast<const uint4*>(slot + 4096 + 1024 * i + 16 * lane);
  __builtin_amdgcn_sched_barrier(0);
  float part[16];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    const cdna4::half8_t k0 = __builtin_bit_cast(cdna4::half8_t, kr[rr][0]);
    const cdna4::half8_t k1 = __builtin_bit_cast(cdna4::half8_t, kr[rr][1]);
#pragma unroll
    for (int hh = 0; hh < 4; ++hh) {
      float acc = __builtin_fmaf(static_cast<float>(k0[0]), qf[hh][0], 0.0f);
#pragma unroll
      for (int j = 1; j < 8; ++j)
        acc = __builtin_fmaf(static_cast<float>(k0[j]), qf[hh][j], acc);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc = __builtin_fmaf(static_cast<float>(k1[j]), qf[hh][8 + j], acc);
      part[4 * hh + rr] = acc;
    }
  }
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, hq = lane >> 5;
  const float s = unit_softmax_state(st, unit_scores(part), u0, span_end, lane);
  const float p = __builtin_amdgcn_exp2f(s - st.m);  // 0 if masked
  st.l += p;
  pf[4 * rq + (dc & 3u)][4 * hq + (dc >> 2)] = p;
  const unsigned a = lane >> 5;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 p0 = *reinterpret_cast<const float4*>(&pf[2 * i + a][0]);
    const float4 p1 = *reinterpret_cast<const float4*>(&pf[2 * i + a][4]);
    const float pp[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
    const cdna4::half8_t v = __builtin_bit_cast(cdna4::half8_t, vr[i]);
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        st.o[h][e] = __builtin_fmaf(static_cast<float>(v[e]), pp[h], st.o[h][e]);
  }
}

// Cross-wave merge relative to the split's true max M_h = max_w mt_w,h, so the partial is
// exactly (max, sum exp(s - max), sum exp(s - max) v). Each wave sums its two row parities across
// its lane halves, stores the result (in slot 0 of its own ring) and its head statistics, then
// after one barrier every thread produces two float4 chunks of the partial: o = sum_w exp2(m_w,h
// - M_h) o_w. `more` says whether the workgroup runs another item afterwards (its LDS is then
// reused).
template <class Shared>
__device__ __attribute__((always_inline)) inline void write_partial(
    const WaveState& st, Shared& sh, float* part_m, float* part_l, float* part_o,
    std::size_t base, bool more) {
  constexpr int kW = Shared::kWaveCount;
  const unsigned t = threadIdx.x, lane = t & 63u, c = lane & 31u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, hq = lane >> 5;
  {
    float l = st.l + cdna4::dpp_mov<cdna4::kQuadXor1>(st.l);
    l += cdna4::dpp_mov<cdna4::kQuadXor2>(l);  // head total over dc % 4, for this rq
    const unsigned h = 4 * hq + (dc >> 2);
    if ((lane & 3u) == 0)
      sh.stat_l[wave][rq][h] = l;
    if ((lane & 0x13u) == 0) {  // rq = 0, dc % 4 = 0: one lane per head
      sh.stat_m[wave][h] = st.m;
      sh.stat_mt[wave][h] = st.mt;
    }
    // Sum the two row parities (lane c holds parity 0, lane c + 32 parity 1, of the same
    // dimensions) across the wave halves: one v_permlane32_swap per pair of heads (h, h + 4)
    // leaves heads 0-3 in the lower half and heads 4-7 in the upper half, summed.
    const unsigned a = lane >> 5;
#pragma unroll
    for (int hh = 0; hh < kGroup / 2; ++hh) {
      float sum[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const cdna4::Pair pr = cdna4::swap32(st.o[hh][e], st.o[hh + kGroup / 2][e]);
        sum[e] = pr.a + pr.b;
      }
      float4* dst =
          reinterpret_cast<float4*>(sh.merge_rows(wave) + (4 * a + hh) * attn::kDim + 8 * c);
      dst[0] = float4{sum[0], sum[1], sum[2], sum[3]};
      dst[1] = float4{sum[4], sum[5], sum[6], sum[7]};
    }
  }
  __syncthreads();
  {
    // 8 heads x 256 floats = 512 float4 chunks; thread t makes chunks t + kThreads j (heads
    // (t + kThreads j) / 64). All LDS reads are issued before any arithmetic (no branches), so
    // the phase costs one LDS round trip.
    constexpr unsigned kChunks = kGroup * attn::kDim / 4, kThreads = kW * 64;
    constexpr unsigned kPer = kChunks / kThreads, kHeadChunks = attn::kDim / 4;
    static_assert(kChunks % kThreads == 0, "chunks per thread");
    float4* dst = reinterpret_cast<float4*>(part_o + base * kGroup * attn::kDim);
    float m[kPer][kW], mt[kPer][kW], lw[kPer][kW];
    float4 x[kPer][kW];
#pragma unroll
    for (unsigned j = 0; j < kPer; ++j) {
      const unsigned i = t + kThreads * j, h = i / kHeadChunks;
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        m[j][w] = sh.stat_m[w][h];
        mt[j][w] = sh.stat_mt[w][h];
        lw[j][w] = sh.stat_l[w][0][h] + sh.stat_l[w][1][h];
        x[j][w] = reinterpret_cast<const float4*>(sh.merge_rows(w))[i];
      }
    }
#pragma unroll
    for (unsigned j = 0; j < kPer; ++j) {
      const unsigned i = t + kThreads * j, h = i / kHeadChunks;
      float M = mt[j][0];
#pragma unroll
      for (int w = 1; w < kW; ++w)
        M = fmaxf(M, mt[j][w]);
      const bool empty = M == -__builtin_inff();  // no key in the span
      const float Mc = empty ? 0.0f : M;          // exp2(-inf - 0) = 0 for every wave
      float4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
      float L = 0.0f;
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        const float sc = __builtin_amdgcn_exp2f(m[j][w] - Mc);
        const float4 x0 = x[j][w];
        acc.x = __builtin_fmaf(sc, x0.x, acc.x);
        acc.y = __builtin_fmaf(sc, x0.y, acc.y);
        acc.z = __builtin_fmaf(sc, x0.z, acc.z);
        acc.w = __builtin_fmaf(sc, x0.w, acc.w);
        L = __builtin_fmaf(sc, lw[j][w], L);
      }
      dst[i] = acc;
      if (i % kHeadChunks == 0) {
        part_m[base * kGroup + h] = M * kLn2;  // -inf stays -inf for an empty span
        part_l[base * kGroup + h] = L;
      }
    }
  }
  if (more)
    __syncthreads();  // LDS is reused by the next item
}

// Where the K/V rows of one sequence and KV head lie. LinearRows: row r at K / V + 256 r.
// PagedRows: rows in pages of 2^log2_page rows; page j of the sequence is page table[j] of the
// pool, which holds [2 KV heads][2^log2_page][256] per page (head_off selects the KV head). An
// 8-row unit never crosses a page (units start at multiples of 8, pages hold >= 8 rows).
struct LinearRows {
  const attn::half_t* K;
  const attn::half_t* V;
};
struct PagedRows {
  const attn::half_t* k_pages;
  const attn::half_t* v_pages;
  const int32_t* table;     // this sequence's page table
  unsigned log2_page;       // rows per page = 1 << log2_page, >= 3
  std::size_t page_halves;  // 2 << log2_page rows of 256 halves: one page of both KV heads
  std::size_t head_off;     // kvh << log2_page rows of 256 halves
};

// Partial (m, l, o) for KV head kvh, written at `base` (= kvh * n_splits + split) in the
// reference's partial layout, over the rows of groups of kW units: the group starting at row
// span.begin and every `stride` rows after it, up to row span.end (rows past it are masked).
// Every caller passes stride = kW * 8, i.e. the contiguous span [span.begin, span.end) (a
// variant whose splits took interleaved 32-row groups, so that all workgroups stream
// neighbouring parts of the cache, measured no faster). Wave w streams unit w of each group
// through its R-unit LDS ring (R - 1 units in flight while one is processed); the waves merge
// through LDS at the end. Every vector-memory load of the kernel is a direct LDS load with an
// explicit wait, except the paged layout's page-table slice, which is waited for before the
// first unit is issued. `more` says whether the workgroup runs another item afterwards (its LDS
// is then reused).
template <DecodeArith kArith, class Shared, class Rows>
__device__ __attribute__((always_inline)) inline void split_partial_rows(
    const float* __restrict__ q, const Rows& rows, unsigned len, AttnSpan span, unsigned stride,
    unsigned kvh, float* part_m, float* part_l, float* part_o, std::size_t base, Shared& sh,
    bool more) {
  constexpr int kW = Shared::kWaveCount, kR = Shared::kRingUnits;
  static_assert(kR >= 2 && kR <= 4 && kGroup % kW == 0, "ring depth / wave count");
  const unsigned t = threadIdx.x, lane = t & 63u, c = lane & 31u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned last_row = len - 1;
  const unsigned kStride = stride;
  const unsigned first = span.begin + wave * kAttnDecodeUnit;
  const unsigned n_units = first < span.end ? (span.end - first + kStride - 1) / kStride : 0;
  const unsigned ring0 = cdna4::lds_offset(sh.ring[wave][0]);
  std::size_t lane_at = 0;
  int tab = 0;
  unsigned page0 = 0;
  if constexpr (std::is_same_v<Rows, LinearRows>) {
    // This lane's address of row pair 0 of unit 0; unit k is kStride rows further.
    lane_at = std::size_t{first + (lane >> 5)} * attn::kDim + c * 8;
  } else {
    // The span's pages, one per lane (a span of at most 64 pages; further pages are read from
    // the table directly).
    page0 = span.begin >> rows.log2_page;
    const unsigned npages =
        span.end > span.begin ? ((span.end - 1) >> rows.log2_page) - page0 + 1 : 0;
    tab = lane < npages ? rows.table[page0 + lane] : 0;
    lane_at = std::size_t{lane >> 5} * attn::kDim + c * 8;
  }
  const std::size_t kUnitStep = std::size_t{kStride} * attn::kDim;
  auto issue = [&](unsigned k) {
    const unsigned u0 = first + k * kStride;
    const unsigned slot = ring0 + (k % kR) * kUnitBytes;
    if constexpr (std::is_same_v<Rows, LinearRows>) {
      if (u0 + kAttnDecodeUnit <= len)  // wave-uniform
        issue_unit(rows.K + lane_at + k * kUnitStep, rows.V + lane_at + k * kUnitStep, slot);
      else
        issue_unit_clamped(rows.K, rows.V, u0, last_row, slot, lane);
    } else {
      const unsigned j = (u0 >> rows.log2_page) - page0;  // wave-uniform
      const int page = j < 64 ? __builtin_amdgcn_readlane(tab, j) : rows.table[page0 + j];
      const unsigned in_page = u0 & ((1u << rows.log2_page) - 1u);
      const std::size_t pg = std::size_t(static_cast<unsigned>(page)) * rows.page_halves +
                             rows.head_off;
      if (u0 + kAttnDecodeUnit <= len) {
        const std::size_t at = pg + std::size_t{in_page} * attn::kDim + lane_at;
        issue_unit(rows.k_pages + at, rows.v_pages + at, slot);
      } else {  // the unit holds the last row: same page
        issue_unit_clamped(rows.k_pages + pg, rows.v_pages + pg, in_page,
                           in_page + (last_row - u0), slot, lane);
      }
    }
  };

  // This wave's query heads of the KV head (1 KiB each), then the first kR - 1 units.
  constexpr int kHeadsPerWave = kGroup / kW;
#pragma unroll
  for (int i = 0; i < kHeadsPerWave; ++i) {
    const unsigned h = kHeadsPerWave * wave + i;
    cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                      cdna4::lds_offset(sh.q[h]));
  }
#pragma unroll
  for (unsigned k = 0; k + 1 < kR; ++k)
    if (k < n_units)
      issue(k);
  wait_units_after(n_units < kR - 1 ? n_units : kR - 1);  // the query loads are older
  __syncthreads();

  // The lane's query slice pre-scaled by log2(e)/16 (1/sqrt(256) in log2 units): slot hh = head
  // 4 hq + (hh ^ dc / 4), dimensions 8 dc .. 8 dc + 7 and 128 + 8 dc .. 128 + 8 dc + 7. In f32
  // (qf[hh][j], j < 8 the first run) or as f16 pairs (qh[hh][p], pairs 0-3 the first run).
  const unsigned dc = lane & 15u, rq = (lane >> 4) & 1u, hq = lane >> 5;
  constexpr bool kF32 = kArith == DecodeArith::kF32;
  constexpr float kScale = kLog2e / 16.0f;
  float qf[4][16];
  half2_t qh[4][8];
#pragma unroll
  for (int hh = 0; hh < 4; ++hh) {
    const unsigned h = 4 * hq + (hh ^ (dc >> 2));
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const float4 x0 = *reinterpret_cast<const float4*>(&sh.q[h][128 * half + 8 * dc]);
      const float4 x1 = *reinterpret_cast<const float4*>(&sh.q[h][128 * half + 8 * dc + 4]);
      const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      if constexpr (kF32) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          qf[hh][8 * half + j] = x[j] * kScale;
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          qh[hh][4 * half + j] = half2_t{static_cast<_Float16>(x[2 * j] * kScale),
                                         static_cast<_Float16>(x[2 * j + 1] * kScale)};
      }
    }
  }
  // K read offsets in a slot: row 4 rq + (rr ^ dc % 4), 16-byte chunk dc (and dc + 16, +256 B).
  unsigned koff[4];
#pragma unroll
  for (int rr = 0; rr < 4; ++rr)
    koff[rr] = (4 * rq + (rr ^ (dc & 3u))) * 512 + 16 * dc;

  WaveState st;
  st.m = -__builtin_inff();
  st.mt = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int h = 0; h < kGroup; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      st.o[h][e] = 0.0f;

  // Steady state: one unit issued and one consumed per iteration, a fixed wait. Its slot held
  // unit k - 1, already read back into registers.
  auto unit = [&](unsigned k) {
    if constexpr (kF32)
      process_unit_f32(st, sh.ring[wave][k % kR], koff, qf, first + k * kStride, span.end,
                       sh.pf[wave], lane);
    else
      process_unit(st, sh.ring[wave][k % kR], koff, qh, first + k * kStride, span.end,
                   sh.p[wave], lane);
  };
  unsigned k = 0;
  for (; k + kR - 1 < n_units; ++k) {
    issue(k + kR - 1);
    cdna4::wait_vmcnt<8 * (kR - 1)>();
    unit(k);
  }
  // Drain: the last units, already in flight.
  for (; k < n_units; ++k) {
    wait_units_after(n_units - 1 - k);
    unit(k);
  }

  write_partial(st, sh, part_m, part_l, part_o, base, more);
}

template <DecodeArith kArith, class Shared>
__device__ __attribute__((always_inline)) inline void split_partial(
    const float* __restrict__ q, const attn::half_t* K, const attn::half_t* V, unsigned len,
    AttnSpan span, unsigned stride, unsigned kvh, float* part_m, float* part_l, float* part_o,
    std::size_t base, Shared& sh, bool more) {
  split_partial_rows<kArith>(q, LinearRows{K, V}, len, span, stride, kvh, part_m, part_l, part_o,
                             base, sh, more);
}

// ------------------------------------------------------------------------------------------------
// The f32-precision split on the matrix cores.
//
// Products: every key is f16 (exact in f32), the query and the softmax numerators are f32. Each
// f32 operand x is carried as the f16 pair (hi, lo) = (f16(x), f16((x - hi) 2^11)), so x = hi +
// 2^-11 lo to ~2^-22 relative, and hi * k, lo * k are exact f32 products. The 8 query heads of
// a KV head times (hi, lo) are exactly the 16 columns of v_mfma_f32_16x16x32_f16: column h holds
// head h's hi part, column 8 + h its lo part, so one MFMA computes both products of every head
// and the two columns are joined as s = hi + 2^-11 lo (lane c and lane c ^ 8 of a row, one DPP
// move). The same holds for O += V^T P^T with the numerators' (hi, lo) as the columns.
//
// Schedule per split workgroup (4 waves): 32-key tiles of K and V stream into a 4-stage LDS ring
// by direct global -> LDS loads (each wave copies 8 rows of each tensor, 1 KiB per instruction),
// one barrier per tile. Every wave computes each tile's scores and softmax decisions itself, so
// the four waves hold identical (m, l) without exchanging anything, and each wave owns 64 of the
// 256 value dimensions of O -- there is no cross-wave merge. The loop is software-pipelined:
// iteration t issues the 16 score MFMAs of tile t + 1 and, between them, the VALU softmax of tile
// t (whose scores the previous iteration produced), then the 4 P V MFMAs of tile t. Tiles t and
// t + 1 are in use and t + 2, t + 3 in flight.
//
// LDS layouts (16-byte chunk c of tile row r at chunk position c ^ s(r) of the row):
//   K: s(r) = r % 16. The A operand read (ds_read_b128) of 16 lanes takes one chunk of 16
//      consecutive rows: 16 distinct positions mod 16.
//   V: s(r) = 2 (r % 8). A transpose read (ds_read_b64_tr_b16) of 32 lanes takes 32 bytes (one
//      16-dimension block) of 8 rows: 8 distinct 32-byte bank groups.
// Operand layouts of the 16x16x32 MFMA (lane l, g = l / 16, c = l % 16; the k index 8 g + j):
//   S^T = K Q^T: A = K rows 16 kb + c, dimensions 8 (4 s + g) + j at k-step s; B = column c of
//     the query pairs over the same dimensions; the result holds keys 16 kb + 4 g + i, column c.
//   O^T += V^T P^T: k-slot 8 g + j is key 4 g + j (j < 4) or 16 + 4 g + j - 4 (j >= 4) of the
//     tile -- exactly the keys of the lane's two score results, so each lane's numerators are its
//     own B operand; A = V^T of dimensions 16 blk + c over those keys (two transpose reads).
// ------------------------------------------------------------------------------------------------

constexpr unsigned kTileKeys = 32;
constexpr unsigned kTileStages = 4;
constexpr unsigned kTileBytes = kTileKeys * attn::kDim * 2;  // 16 KiB per K or V tile
constexpr float kLoScale = 2048.0f;                          // 2^11: the lo half of a pair
constexpr float kLoWeight = 1.0f / 2048.0f;
constexpr int kSc1 = 16;  // cache-policy operand of the buffer builtins: sc1 (agent-coherent)

// K tiles in the first 64 KiB (so a K operand address plus its stage offset stays under the
// 16-bit instruction offset), V tiles in the next 64 KiB, then the KV head's 8 query rows.
struct alignas(1024) TileShared {
  unsigned char k[kTileStages][kTileBytes];
  unsigned char v[kTileStages][kTileBytes];
  float q[kGroup][attn::kDim];
};

__device__ inline unsigned tile_swz_k(unsigned row, unsigned chunk) { return chunk ^ (row & 15u); }
__device__ inline unsigned tile_swz_v(unsigned row, unsigned chunk) {
  return chunk ^ (2u * (row & 7u));
}

typedef cdna4::float4_t f32x4;

__device__ __attribute__((always_inline)) inline f32x4 mfma16(const cdna4::half8_t& a,
                                                             const cdna4::half8_t& b,
                                                             const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __attribute__((always_inline)) inline cdna4::half8_t lds_b128(unsigned addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) cdna4::half8_t*>(addr);
}

typedef __fp16 tile_fp16x4 __attribute__((vector_size(8)));
__device__ __attribute__((always_inline)) inline cdna4::half4_t lds_tr_b64(unsigned addr) {
  const tile_fp16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      reinterpret_cast<__attribute__((address_space(3))) tile_fp16x4*>(addr));
  return __builtin_bit_cast(cdna4::half4_t, raw);
}

// A workgroup barrier that waits only for this wave's LDS reads: the tiles in flight (direct LDS
// loads, counted by vmcnt) stay in flight across it. A compiler memory barrier on both sides.
__device__ __attribute__((always_inline)) inline void tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until this wave's copy of the tile followed by `after` (< 3) more tile copies has landed
// (8 instructions per tile copy).
__device__ __attribute__((always_inline)) inline void wait_tiles_after(unsigned after) {
  switch (after) {
    case 0: cdna4::wait_vmcnt<0>(); break;
    case 1: cdna4::wait_vmcnt<8>(); break;
    default: cdna4::wait_vmcnt<16>(); break;
  }
}

// Copy of this wave's 8 rows of a K and a V tile whose rows all exist: instruction i moves rows
// 8 w + 2 i + lane / 32 of the tile, LDS chunk position lane % 32 <- the row's chunk at that
// position's swizzle. kt / vt: the wave's first row (wave-uniform); koff[i] / voff[i]: the lane's
// byte offset from it minus 1024 i, since the instruction offset (1024 i) moves the global and the
// LDS address alike. The loads carry the non-temporal hint (the cache is streamed once per call).
// M0 is saved and restored.
__device__ __attribute__((always_inline)) inline void issue_rows8(const void* kt, const void* vt,
                                                                 const unsigned (&koff)[4],
                                                                 const unsigned (&voff)[4],
                                                                 unsigned k_lds, unsigned v_lds) {
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
      : "v"(koff[0]), "v"(koff[1]), "v"(koff[2]), "v"(koff[3]), "v"(voff[0]), "v"(voff[1]),
        "v"(voff[2]), "v"(voff[3]), "s"(kt), "s"(vt), "s"(k_lds), "s"(v_lds)
      : "memory");
}

// Where the rows of a split lie, for the tile copies: k_at(row) / v_at(row) is the address of K /
// V row `row`, valid for the 8-row group (aligned to 8) that holds it.
struct LinearTiles {
  const attn::half_t* K;
  const attn::half_t* V;
  __device__ const attn::half_t* k_at(unsigned row) const { return K + std::size_t{row} * attn::kDim; }
  __device__ const attn::half_t* v_at(unsigned row) const { return V + std::size_t{row} * attn::kDim; }
};
// Paged rows: the pages of the split's rows, one per lane from page0 (at most 64; a page past
// them is read from the table), read with a uniform readlane.
struct PagedTiles {
  PagedRows rows;
  int tab;
  unsigned page0;
  __device__ std::size_t at(unsigned row) const {
    const unsigned j = (row >> rows.log2_page) - page0;  // wave-uniform
    const int page = j < 64 ? __builtin_amdgcn_readlane(tab, j) : rows.table[page0 + j];
    return std::size_t(static_cast<unsigned>(page)) * rows.page_halves + rows.head_off +
           std::size_t{row & ((1u << rows.log2_page) - 1u)} * attn::kDim;
  }
  __device__ const attn::half_t* k_at(unsigned row) const { return rows.k_pages + at(row); }
  __device__ const attn::half_t* v_at(unsigned row) const { return rows.v_pages + at(row); }
};

// A wave-uniform address, in scalar registers (the copies take their base there).
__device__ __attribute__((always_inline)) inline const attn::half_t* uniform(const attn::half_t* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  return reinterpret_cast<const attn::half_t*>((uint64_t{hi} << 32) | lo);
}

// This wave's 8 rows of the tile at key k0 into the K and V slots k_lds / v_lds (this wave's 4 KiB
// of each): rows past last_row read last_row instead (they are masked at use), so no load
// leaves the split's rows. Always 8 vector-memory instructions.
template <class Tiles>
__device__ __attribute__((always_inline)) inline void issue_tile(
    const Tiles& tl, unsigned k0, unsigned last_row, unsigned k_lds, unsigned v_lds,
    const unsigned (&koff)[4], const unsigned (&voff)[4], unsigned wave, unsigned lane) {
  const unsigned gs = k0 + 8 * wave;  // the group's first row (wave-uniform)
  if (gs + 7 <= last_row) {
    issue_rows8(uniform(tl.k_at(gs)), uniform(tl.v_at(gs)), koff, voff, k_lds, v_lds);
  } else {
    const unsigned row0 = gs <= last_row ? gs : last_row;
    const unsigned lim = last_row - row0;  // rows of the group past last_row read row0 + lim
    const attn::half_t* K = tl.k_at(row0);
    const attn::half_t* V = tl.v_at(row0);
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
      const unsigned j = 2 * i + (lane >> 5), r = 8 * wave + j, p = lane & 31u;
      const std::size_t at = std::size_t{j < lim ? j : lim} * attn::kDim;
      cdna4::lds_load16_nt(K + at + 8 * tile_swz_k(r, p), k_lds + 1024 * i);
      cdna4::lds_load16_nt(V + at + 8 * tile_swz_v(r, p), v_lds + 1024 * i);
    }
  }
}

// Per-lane state of a wave over its split (lane l, g = l / 16, c = l % 16, head h = c % 8).
//   q[s]: B operand of k-step s: head h's query x log2(e)/16, dimensions 8 (4 s + g) + j, as
//         its hi (c < 8) or lo (c >= 8) f16 half.
//   m: the reference max of head h (log2 units, 0 before the first tile), moved lazily;
//   mt: the true max; l: the sum of this lane's numerators (keys 4 g + i and 16 + 4 g + i of
//   every tile, relative to m).
//   o[b]: O^T of dimensions 64 w + 16 b + 4 g + i, column c, relative to m.
template <int kBlocks>
struct TileStateT {
  cdna4::half8_t q[8];
  float m, mt, l;
  f32x4 o[kBlocks];
};
using TileState = TileStateT<4>;

// The K operands of one tile (both 16-key blocks, 8 k-steps): ka[kb][s] at (kaddr + 8192 kb) ^
// 64 s, kaddr = the tile's K slot + the lane's offset.
__device__ __attribute__((always_inline)) inline void read_k(cdna4::half8_t (&ka)[2][8],
                                                            unsigned kaddr) {
#pragma unroll
  for (unsigned s = 0; s < 8; ++s)
#pragma unroll
    for (unsigned kb = 0; kb < 2; ++kb)
      ka[kb][s] = lds_b128((kaddr + 8192u * kb) ^ (64u * s));
}

// The V^T operands of this wave's 4 dimension blocks (two transpose reads each: rows 4 g + r and
// 16 + 4 g + r).
__device__ __attribute__((always_inline)) inline void read_v(cdna4::half8_t (&va)[4],
                                                            unsigned vslot,
                                                            const unsigned (&vl)[4]) {
#pragma unroll
  for (unsigned b = 0; b < 4; ++b) {
    const cdna4::half4_t lo = lds_tr_b64(vslot + vl[b]);
    const cdna4::half4_t up = lds_tr_b64(vslot + vl[b] + 8192u);
    va[b] = cdna4::half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
  }
}

// Score MFMA k-step s of both key blocks.
__device__ __attribute__((always_inline)) inline void score_step(f32x4 (&s)[2],
                                                                const cdna4::half8_t (&ka)[2][8],
                                                                const cdna4::half8_t& q,
                                                                unsigned step) {
  if (step == 0) {
    s[0] = mfma16(ka[0][0], q, f32x4{});
    s[1] = mfma16(ka[1][0], q, f32x4{});
  } else {
    s[0] = mfma16(ka[0][step], q, s[0]);
    s[1] = mfma16(ka[1][step], q, s[1]);
  }
}

// The softmax of one tile, in log2 units relative to the reference max m of the lane's head.
// The (hi, lo) columns are joined in every lane (lane c and lane c ^ 8 both form hi + 2^-11 lo
// of head c % 8) with m subtracted in the same instructions; keys k0 + key >= lim are masked when
// kMasked. The numerators 2^x are speculated with the current m; the reference max moves (the
// caller runs tile_rescale before using them) when the tile's head max exceeds m by more than
// the slack in any lane, and always on the split's first tile, whose max becomes m.
struct TileSoftmax {
  float x[8];    // scores minus m, -inf where masked
  float mx, lt;  // the tile's head max of x; the sum of the numerators
  cdna4::half8_t pb;
};

// Per-lane constants of the pair columns: the join weights (hi lanes 1 and 2^-11 for their own
// and the partner's accumulator, lo lanes the reverse) and the split of a value x with hi =
// f16(x) into this lane's half r = f16(hi a + x b): hi itself in the hi lanes (a = 1, b = 0: hi 1
// + 0 is exact, so the hi lanes return the very value the lo lanes subtract, however the compiler
// rounded it), the lo half f16((x - hi) 2^11) in the lo lanes (a = -2^11, b = 2^11): one
// expression, no select.
struct TileLane {
  float w_own, w_other, a, b;
};
__device__ __attribute__((always_inline)) inline TileLane tile_lane(unsigned lane) {
  const bool is_hi = (lane & 15u) < 8;
  return is_hi ? TileLane{1.0f, kLoWeight, 1.0f, 0.0f}
               : TileLane{kLoWeight, 1.0f, -kLoScale, kLoScale};
}

// This lane's half of the pair of x, given hi = f16(x).
__device__ __attribute__((always_inline)) inline _Float16 pair_half(_Float16 hi, float x,
                                                                   const TileLane& tl) {
  return static_cast<_Float16>(__builtin_fmaf(static_cast<float>(hi), tl.a, x * tl.b));
}

// max(a, b) and max(a, b, c) without canonicalising the inputs (scores are never NaN).
__device__ __attribute__((always_inline)) inline float tile_max(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __attribute__((always_inline)) inline float tile_max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// x = (own w_own + partner w_other) kscale - m. own w_own is exact (a power of two), and one
// v_fmac adds the partner (lane ^ 8) read through DPP, so both lanes of a pair round the same
// exact sum hi + 2^-11 lo once and hold identical x: the pair's hi and lo halves of each
// numerator are then cut from the same value. kscale: the keys' K row scales (kKScale), else 1.
// The leading s_nop gives the DPP source reads the two wait states they need after a VALU write.
template <bool kMasked, bool kKScale = false>
__device__ __attribute__((always_inline)) inline void tile_scores_joined(
    TileSoftmax& sm, const f32x4 (&s)[2], float m, unsigned k0, unsigned lim, unsigned lane,
    const TileLane& tl, const float* kscale = nullptr) {
  float own[8], t[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    own[i] = s[i / 4][i % 4];
    t[i] = own[i] * tl.w_own;
  }
  asm volatile(
      "s_nop 1\n\t"
      "v_fmac_f32_dpp %0, %8, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %1, %9, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %2, %10, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %3, %11, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %4, %12, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %5, %13, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %6, %14, %16 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "v_fmac_f32_dpp %7, %15, %16 row_ror:8 row_mask:0xf bank_mask:0xf"
      : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]), "+v"(t[4]), "+v"(t[5]), "+v"(t[6]),
        "+v"(t[7])
      : "v"(own[0]), "v"(own[1]), "v"(own[2]), "v"(own[3]), "v"(own[4]), "v"(own[5]),
        "v"(own[6]), "v"(own[7]), "v"(tl.w_other));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (kKScale)
      sm.x[i] = __builtin_fmaf(t[i], kscale[i], -m);
    else
      sm.x[i] = t[i] - m;
  }
  if constexpr (kMasked) {
    const unsigned g = lane >> 4;
#pragma unroll
    for (unsigned i = 0; i < 8; ++i) {
      const unsigned key = k0 + (i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4));
      sm.x[i] = key < lim ? sm.x[i] : -__builtin_inff();
    }
  }
}

// The numerators p = 2^(x - shift) (times vr, the V row scale ratios, when kV), their sum (of the
// unscaled p) and this lane's half of each as the P^T operand.
template <bool kV>
__device__ __attribute__((always_inline)) inline void tile_numerators(TileSoftmax& sm, float shift,
                                                                     const TileLane& tl,
                                                                     const float* vr) {
  _Float16 ph[8];
  float lt = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    float p0 = __builtin_amdgcn_exp2f(sm.x[i] - shift);  // 0 if masked
    float p1 = __builtin_amdgcn_exp2f(sm.x[i + 1] - shift);
    lt += p0;
    lt += p1;
    if constexpr (kV) {
      p0 *= vr[i];
      p1 *= vr[i + 1];
    }
    const cdna4::half2_t h{static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
    ph[i] = pair_half(h[0], p0, tl);
    ph[i + 1] = pair_half(h[1], p1, tl);
  }
  sm.lt = lt;
  sm.pb = cdna4::half8_t{ph[0], ph[1], ph[2], ph[3], ph[4], ph[5], ph[6], ph[7]};
}

// Head max over the tile (the lane's 8 keys, then the 4 lanes g of its column; every tile has a
// key in the split, so it is finite), the true max, and the speculative numerators. `first`:
// the split's first tile (wave-uniform).
template <bool kV = false, int kBlocks = 4>
__device__ __attribute__((always_inline)) inline bool tile_decide(TileSoftmax& sm,
                                                                 TileStateT<kBlocks>& st,
                                                                 bool first, const TileLane& tl,
                                                                 const float* vr = nullptr) {
  const float* x = sm.x;
  float mx = tile_max3(tile_max3(x[0], x[1], x[2]), tile_max3(x[3], x[4], x[5]),
                       tile_max(x[6], x[7]));
  {
    const cdna4::Pair a = cdna4::swap16(mx, mx);
    mx = tile_max(a.a, a.b);
    const cdna4::Pair b = cdna4::swap32(mx, mx);
    mx = tile_max(b.a, b.b);
  }
  sm.mx = mx;
  st.mt = fmaxf(st.mt, mx + st.m);
  tile_numerators<kV>(sm, 0.0f, tl, vr);
  return first || __builtin_amdgcn_ballot_w64(mx > kRescaleSlack) != 0;
}

// O *= c for accumulators in AGPRs, in place (the copies through a VGPR stay inside the rarely
// taken branch; as C++, the compiler hoists copies of O out of it to every iteration). The
// leading no-ops let the last P V MFMA's results settle; the trailing ones separate the AGPR
// writes from the next MFMA reading them.
template <int kBlocks>
__device__ __attribute__((always_inline)) inline void tile_scale_o(f32x4 (&o)[kBlocks], float c) {
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int b = 0; b < kBlocks; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x = o[b][i], tmp;
      asm volatile(
          "v_accvgpr_read_b32 %1, %0\n\t"
          "v_mul_f32 %1, %1, %2\n\t"
          "v_accvgpr_write_b32 %0, %1"
          : "+a"(x), "=&v"(tmp)
          : "v"(c));
      o[b][i] = x;
    }
  asm volatile("s_nop 3" ::: "memory");
}

// The rare path: move the reference max of each head by d = max(0, tile max) (the tile max on
// the first tile), rescale l and O, and redo the numerators.
template <bool kV = false, int kBlocks = 4>
__device__ __attribute__((always_inline)) inline void tile_rescale(TileSoftmax& sm,
                                                                  TileStateT<kBlocks>& st,
                                                                  bool first, const TileLane& tl,
                                                                  const float* vr = nullptr) {
  const float d = first ? sm.mx : fmaxf(sm.mx, 0.0f);
  const float corr = first ? 0.0f : __builtin_amdgcn_exp2f(-d);  // l and O are 0 on the first
  st.m += d;
  st.l *= corr;
  tile_scale_o(st.o, corr);
  tile_numerators<kV>(sm, d, tl, vr);
}

// Partial (m, l, o) of KV head kvh over keys [span.begin, span.end) (span.end <= len), written at
// `base` (= kvh * n_splits + split, or the batched paths' index) in the reference's partial
// layout: m in natural-log units, l and o relative to the split's true max (an empty span
// writes m = -inf, l = 0, o = 0). Every vector-memory load of the stream is a direct LDS load
// with an explicit wait. `more` says whether the workgroup runs another item afterwards (its LDS
// is then reused).
// kCoherent: the partial is stored with agent-coherent accesses (cache policy sc1, what a relaxed
// agent-scope atomic access compiles to on gfx950), so a workgroup on another XCD can read it
// after a counter hand-off (attn_decode_fused_kernel); `part_floats` bounds those stores.
template <class Tiles, bool kCoherent = false>
__device__ __attribute__((always_inline)) inline void split_partial_tiles(
    const float* __restrict__ q, const Tiles& tl, AttnSpan span, unsigned kvh, float* part_m,
    float* part_l, float* part_o, std::size_t base, TileShared& sh, bool more,
    unsigned part_floats = 0) {
  using cdna4::half8_t;
  const unsigned t = threadIdx.x, lane = t & 63u, g = lane >> 4, c = lane & 15u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned n_tiles = (span.end - span.begin + kTileKeys - 1) / kTileKeys;
  const unsigned last_row = span.end - 1;  // unused when n_tiles == 0
  const unsigned k_lds0 = cdna4::lds_offset(sh.k[0]) + 4096 * wave;
  const unsigned v_lds0 = cdna4::lds_offset(sh.v[0]) + 4096 * wave;

  // Copy offsets: instruction i moves tile row r = 8 w + 2 i + lane / 32 (row j = r - 8 w of the
  // wave's group), LDS chunk position lane % 32.
  unsigned koff[4], voff[4];
#pragma unroll
  for (unsigned i = 0; i < 4; ++i) {
    const unsigned j = 2 * i + (lane >> 5), r = 8 * wave + j, p = lane & 31u;
    koff[i] = j * 512 + 16 * tile_swz_k(r, p) - 1024 * i;
    voff[i] = j * 512 + 16 * tile_swz_v(r, p) - 1024 * i;
  }
  auto issue = [&](unsigned ti) __attribute__((always_inline)) {
    const unsigned stage = ti % kTileStages;
    issue_tile(tl, span.begin + ti * kTileKeys, last_row, k_lds0 + stage * kTileBytes,
               v_lds0 + stage * kTileBytes, koff, voff, wave, lane);
  };

  // The KV head's 8 query rows (wave w: rows 2 w, 2 w + 1), then the first three tiles.
#pragma unroll
  for (unsigned i = 0; i < 2; ++i) {
    const unsigned h = 2 * wave + i;
    cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                      cdna4::lds_offset(sh.q[h]));
  }
#pragma unroll
  for (unsigned ti = 0; ti < kTileStages - 1; ++ti)
    if (ti < n_tiles)
      issue(ti);

  // Operand offsets. K: row 16 kb + c, chunk 4 s + g at position (4 s + g) ^ c, i.e. byte
  // 512 c + 16 (g ^ c % 4) + 64 (s ^ c / 4) = kl ^ 64 s (+ 8192 kb; the slot base has no bits
  // below 14). V^T: lane 16 g + 4 r + e reads row 4 g + r, dimensions 16 blk + 4 e .. + 3 (blk =
  // 4 w + b): chunk 2 blk + e / 2 at position 2 (blk ^ row % 8) + e / 2.
  const unsigned kl = 512 * c + 16 * (g ^ (c & 3u)) + 64 * (c >> 2);
  unsigned vl[4];
  {
    const unsigned r = (lane >> 2) & 3u, e = lane & 3u, row = 4 * g + r;
#pragma unroll
    for (unsigned b = 0; b < 4; ++b)
      vl[b] = 512 * row + 32 * ((4 * wave + b) ^ (row & 7u)) + 8 * e;
  }
  auto kslot = [&](unsigned ti) __attribute__((always_inline)) {
    return cdna4::lds_offset(sh.k[ti % kTileStages]) + kl;
  };
  auto vslot = [&](unsigned ti) __attribute__((always_inline)) {
    return cdna4::lds_offset(sh.v[ti % kTileStages]);
  };

  TileState st;
  st.m = 0.0f;
  st.mt = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    st.o[b] = f32x4{};
  f32x4 s_cur[2] = {f32x4{}, f32x4{}};
  const TileLane tln = tile_lane(lane);

  if (n_tiles > 0) {
    wait_tiles_after(n_tiles - 1 < 2 ? n_tiles - 1 : 2);  // tile 0 and the queries landed
    tile_barrier();
    // Query pairs: head c % 8, dimensions 8 (4 s + g) .. + 7, x log2(e)/16 (1/sqrt(256) in
    // log2 units), hi half in columns 0-7, lo half in columns 8-15 (pair_half's split).
    const float* qrow = sh.q[c & 7u];
    constexpr float kScale = kLog2e / 16.0f;
#pragma unroll
    for (unsigned s = 0; s < 8; ++s) {
      const float4 x0 = *reinterpret_cast<const float4*>(qrow + 8 * (4 * s + g));
      const float4 x1 = *reinterpret_cast<const float4*>(qrow + 8 * (4 * s + g) + 4);
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      _Float16 hv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = xs[j] * kScale;
        hv[j] = pair_half(static_cast<_Float16>(v), v, tln);
      }
      st.q[s] = half8_t{hv[0], hv[1], hv[2], hv[3], hv[4], hv[5], hv[6], hv[7]};
    }
    half8_t ka[2][8];
    read_k(ka, kslot(0));
#pragma unroll
    for (unsigned s = 0; s < 8; ++s)
      score_step(s_cur, ka, st.q[s], s);
  }

  // Iteration ti < n_tiles - 1: tile ti + 1 lands (this wave's copy by vmcnt, every wave's by the
  // barrier, which also says that every wave is done with tile ti - 1, whose stage then receives
  // tile ti + 3). The 16 score MFMAs of tile ti + 1 go to the matrix cores interleaved with the
  // VALU softmax of tile ti, whose scores the previous iteration produced; then O += V^T P^T of
  // tile ti. The last tile has no successor: its softmax and P V alone.
  auto softmax_pv = [&](const half8_t (&va)[4], TileSoftmax& sm, bool moved, bool first)
      __attribute__((always_inline)) {
    if (moved)
      tile_rescale(sm, st, first, tln);
    st.l += sm.lt;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      st.o[b] = mfma16(va[b], sm.pb, st.o[b]);
  };
  auto join = [&](unsigned ti, TileSoftmax& sm) __attribute__((always_inline)) {
    const unsigned k0 = span.begin + ti * kTileKeys;
    if (k0 + kTileKeys > span.end)  // uniform: only the last tile
      tile_scores_joined<true>(sm, s_cur, st.m, k0, span.end, lane, tln);
    else
      tile_scores_joined<false>(sm, s_cur, st.m, k0, span.end, lane, tln);
  };
  for (unsigned ti = 0; ti + 1 < n_tiles; ++ti) {
    const unsigned ahead = n_tiles - 2 - ti;  // copies issued after tile ti + 1's
    wait_tiles_after(ahead < 1 ? ahead : 1);
    tile_barrier();
    if (ti + kTileStages - 1 < n_tiles)
      issue(ti + kTileStages - 1);  // into tile ti - 1's stage
    TileSoftmax sm;
    join(ti, sm);
    half8_t ka[2][8], va[4];
    read_k(ka, kslot(ti + 1));
    read_v(va, vslot(ti), vl);
    __builtin_amdgcn_sched_barrier(0);  // every operand read in flight before the MFMAs
    f32x4 s_next[2];
#pragma unroll
    for (unsigned s = 0; s < 8; ++s)
      score_step(s_next, ka, st.q[s], s);
    const bool moved = tile_decide(sm, st, ti == 0, tln);
    // The speculative numerators are computed here, between the MFMAs, not sunk past the branch.
    asm volatile("" : "+v"(sm.lt), "+v"(sm.pb));
    // 16 MFMAs, each followed by up to 6 VALU instructions of the softmax.
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    }
    softmax_pv(va, sm, moved, ti == 0);
    s_cur[0] = s_next[0];
    s_cur[1] = s_next[1];
  }
  if (n_tiles > 0) {
    const unsigned ti = n_tiles - 1;
    TileSoftmax sm;
    join(ti, sm);
    half8_t va[4];
    read_v(va, vslot(ti), vl);
    const bool moved = tile_decide(sm, st, ti == 0, tln);
    softmax_pv(va, sm, moved, ti == 0);
  }

  // Relative to the true max; l summed over the lanes g of the column; the (hi, lo) columns of
  // O joined in the lanes c < 8, which store this wave's 64 dimensions of head c.
  const bool empty = n_tiles == 0;
  const float f = empty ? 1.0f : __builtin_amdgcn_exp2f(st.m - st.mt);
  const float L = cdna4::sum_xor32(cdna4::sum_xor16(st.l)) * f;
  const unsigned h = c & 7u;
#pragma unroll
  for (unsigned b = 0; b < 4; ++b) {
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = st.o[b][i] * f;
      o[i] = __builtin_fmaf(cdna4::dpp_mov<cdna4::kRowRor8>(x), kLoWeight, x);
    }
    if (c < 8) {
      const std::size_t at = (base * kGroup + h) * attn::kDim + 64 * wave + 16 * b + 4 * g;
      if constexpr (kCoherent)
        __builtin_amdgcn_raw_buffer_store_b128(
            cdna4::u32x4_t{__builtin_bit_cast(unsigned, o[0]), __builtin_bit_cast(unsigned, o[1]),
                           __builtin_bit_cast(unsigned, o[2]), __builtin_bit_cast(unsigned, o[3])},
            __builtin_amdgcn_make_buffer_rsrc(part_o, 0, static_cast<int>(4 * part_floats),
                                              0x00020000),
            static_cast<int>(4 * at), 0, kSc1);
      else
        *reinterpret_cast<float4*>(part_o + at) = float4{o[0], o[1], o[2], o[3]};
    }
  }
  if (wave == 0 && lane < 8) {
    const float m_nat = st.mt * kLn2;  // -inf stays -inf for an empty span
    if constexpr (kCoherent) {
      __hip_atomic_store(part_m + base * kGroup + h, m_nat, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(part_l + base * kGroup + h, L, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    } else {
      part_m[base * kGroup + h] = m_nat;
      part_l[base * kGroup + h] = L;
    }
  }
  if (more)
    tile_barrier();  // LDS is reused by the next item
}

// ------------------------------------------------------------------------------------------------
// Per-wave tiles. Each wave streams whole 32-key tiles of its own (tiles w, w + 4, ... of an
// item) through its own K and V slot (sh.k[w], sh.v[w]) and keeps its own softmax state with O
// over all 256 dimensions (16 blocks), so no score or softmax is computed twice and the tile
// loop has no workgroup barrier: the next tile's K is issued as soon as this tile's K operands
// are in registers, its V as soon as this tile's V operands are. The four wave states of an
// item are merged in LDS at its end (wave_merge_*).
// ------------------------------------------------------------------------------------------------

// Wait until at most n of this wave's vector-memory instructions are in flight, n rounded down to
// a multiple of 4 and capped at 60 (waiting for more than needed is only slower).
__device__ __attribute__((always_inline)) inline void wait_vm_at_most(unsigned n) {
  switch (n < 60 ? n / 4 : 15) {
    case 0: cdna4::wait_vmcnt<0>(); break;
    case 1: cdna4::wait_vmcnt<4>(); break;
    case 2: cdna4::wait_vmcnt<8>(); break;
    case 3: cdna4::wait_vmcnt<12>(); break;
    case 4: cdna4::wait_vmcnt<16>(); break;
    case 5: cdna4::wait_vmcnt<20>(); break;
    case 6: cdna4::wait_vmcnt<24>(); break;
    case 7: cdna4::wait_vmcnt<28>(); break;
    case 8: cdna4::wait_vmcnt<32>(); break;
    case 9: cdna4::wait_vmcnt<36>(); break;
    case 10: cdna4::wait_vmcnt<40>(); break;
    case 11: cdna4::wait_vmcnt<44>(); break;
    case 12: cdna4::wait_vmcnt<48>(); break;
    case 13: cdna4::wait_vmcnt<52>(); break;
    case 14: cdna4::wait_vmcnt<56>(); break;
    default: cdna4::wait_vmcnt<60>(); break;
  }
}

// Copy of 8 rows of one K or V tile whose rows all exist: instruction i moves rows 2 i + lane / 32
// of the group at xt, LDS chunk position lane % 32 of those rows at lds (`off`: the lane's byte
// offset from xt minus 1024 i, since the instruction offset moves the global and the LDS address
// alike). Non-temporal loads; M0 is saved and restored.
__device__ __attribute__((always_inline)) inline void issue_rows4(const void* xt,
                                                                 const unsigned (&off)[4],
                                                                 unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %6\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %5 nt\n\t"
      "global_load_lds_dwordx4 %2, %5 offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %3, %5 offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %4, %5 offset:3072 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(xt), "s"(lds)
      : "memory");
}

// Copy offsets of a wave's whole-tile copies, in the layout of the tile slots (row r at byte
// 512 r, chunk position p holding chunk tile_swz(r, p)): group g (rows 8 g ..), instruction i,
// row r = 8 g + 2 i + lane / 32. K's swizzle depends on r % 16 (so on g's parity), V's on r % 8.
struct WaveCopy {
  unsigned koff[2][4];
  unsigned voff[4];
};
__device__ __attribute__((always_inline)) inline WaveCopy wave_copy_offsets(unsigned lane) {
  WaveCopy cp;
#pragma unroll
  for (unsigned i = 0; i < 4; ++i) {
    const unsigned j = 2 * i + (lane >> 5), p = lane & 31u;
#pragma unroll
    for (unsigned par = 0; par < 2; ++par)
      cp.koff[par][i] = j * 512 + 16 * tile_swz_k(8 * par + j, p) - 1024 * i;
    cp.voff[i] = j * 512 + 16 * tile_swz_v(j, p) - 1024 * i;
  }
  return cp;
}

// Row `row` of group G of a tile (K: kV false, V: kV true), for the wave copies. Sources whose
// rows need the group (the paged stream's per-tile pages) overload it.
template <bool kV, unsigned G, class Tiles>
__device__ __attribute__((always_inline)) inline const attn::half_t* tile_group_row(
    const Tiles& tl, unsigned row) {
  return kV ? tl.v_at(row) : tl.k_at(row);
}

// Group G (rows 8 G .. 8 G + 7) of this wave's copy of a tile at key k0 into its slot at lds: 4
// vector-memory instructions; rows past last_row read last_row instead (they are masked at use),
// so no load leaves the item's rows.
template <bool kV, unsigned G, class Tiles>
__device__ __attribute__((always_inline)) inline void issue_wave_group(const Tiles& tl,
                                                                      unsigned k0,
                                                                      unsigned last_row,
                                                                      unsigned lds,
                                                                      const WaveCopy& cp,
                                                                      unsigned lane) {
  const unsigned gs = k0 + 8 * G;  // the group's first row (wave-uniform)
  const unsigned(&off)[4] = kV ? cp.voff : cp.koff[G & 1u];
  if (gs + 7 <= last_row) {
    issue_rows4(uniform(tile_group_row<kV, G>(tl, gs)), off, lds + 4096 * G);
  } else {
    const unsigned row0 = gs <= last_row ? gs : last_row;
    const unsigned lim = last_row - row0;  // rows of the group past last_row read row0 + lim
    const attn::half_t* X = tile_group_row<kV, G>(tl, row0);
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
      const unsigned j = 2 * i + (lane >> 5), r = 8 * G + j, p = lane & 31u;
      const std::size_t at = std::size_t{j < lim ? j : lim} * attn::kDim;
      cdna4::lds_load16_nt(X + at + 8 * (kV ? tile_swz_v(r, p) : tile_swz_k(r, p)),
                           lds + 4096 * G + 1024 * i);
    }
  }
}

// This wave's copy of the whole K (kV false) or V (kV true) tile at key k0 into its slot at lds:
// 4 groups of 8 rows, always 16 vector-memory instructions.
template <bool kV, class Tiles>
__device__ __attribute__((always_inline)) inline void issue_wave_tile(const Tiles& tl, unsigned k0,
                                                                     unsigned last_row,
                                                                     unsigned lds,
                                                                     const WaveCopy& cp,
                                                                     unsigned lane) {
  issue_wave_group<kV, 0>(tl, k0, last_row, lds, cp, lane);
  issue_wave_group<kV, 1>(tl, k0, last_row, lds, cp, lane);
  issue_wave_group<kV, 2>(tl, k0, last_row, lds, cp, lane);
  issue_wave_group<kV, 3>(tl, k0, last_row, lds, cp, lane);
}

// The V^T operands of all 16 dimension blocks of a tile (two transpose reads each: rows 4 g + r
// and 16 + 4 g + r). vl[j]: the lane's offset for blocks j and j + 8 (+256 bytes).
__device__ __attribute__((always_inline)) inline void read_v_all(cdna4::half8_t (&va)[16],
                                                                unsigned vslot,
                                                                const unsigned (&vl)[8]) {
#pragma unroll
  for (unsigned b = 0; b < 16; ++b) {
    const unsigned a = vslot + vl[b & 7u] + 256u * (b >> 3);
    const cdna4::half4_t lo = lds_tr_b64(a);
    const cdna4::half4_t up = lds_tr_b64(a + 8192u);
    va[b] = cdna4::half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
  }
}

using WaveTileState = TileStateT<16>;

// Per-lane operand offsets of the wave loops: kl into a K slot (as split_partial_tiles), vl[j]
// into a V slot for dimension blocks j and j + 8.
struct WaveOperands {
  unsigned kl;
  unsigned vl[8];
};
__device__ __attribute__((always_inline)) inline WaveOperands wave_operands(unsigned lane) {
  WaveOperands op;
  const unsigned g = lane >> 4, c = lane & 15u;
  op.kl = 512 * c + 16 * (g ^ (c & 3u)) + 64 * (c >> 2);
  const unsigned r = (lane >> 2) & 3u, e = lane & 3u, row = 4 * g + r;
#pragma unroll
  for (unsigned j = 0; j < 8; ++j)
    op.vl[j] = 512 * row + 32 * (j ^ (row & 7u)) + 8 * e;
  return op;
}

// Fresh state of an item; the query pairs from its f32 rows qrows[8][256] (as split_partial_tiles:
// head c % 8, dimensions 8 (4 s + g) .. + 7, x log2(e)/16, hi half in columns 0-7, lo in 8-15).
__device__ __attribute__((always_inline)) inline void wave_start(WaveTileState& st,
                                                                const float (*qrows)[attn::kDim],
                                                                unsigned lane,
                                                                const TileLane& tln) {
  const unsigned g = lane >> 4, c = lane & 15u;
  st.m = 0.0f;
  st.mt = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int b = 0; b < 16; ++b)
    st.o[b] = f32x4{};
  const float* qrow = qrows[c & 7u];
  constexpr float kScale = kLog2e / 16.0f;
#pragma unroll
  for (unsigned s = 0; s < 8; ++s) {
    const float4 x0 = *reinterpret_cast<const float4*>(qrow + 8 * (4 * s + g));
    const float4 x1 = *reinterpret_cast<const float4*>(qrow + 8 * (4 * s + g) + 4);
    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    _Float16 hv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = xs[j] * kScale;
      hv[j] = pair_half(static_cast<_Float16>(v), v, tln);
    }
    st.q[s] = cdna4::half8_t{hv[0], hv[1], hv[2], hv[3], hv[4], hv[5], hv[6], hv[7]};
  }
}

// The scores of one tile (its K operands already read into ka).
__device__ __attribute__((always_inline)) inline void wave_scores(f32x4 (&s)[2],
                                                                 const cdna4::half8_t (&ka)[2][8],
                                                                 const WaveTileState& st) {
#pragma unroll
  for (unsigned i = 0; i < 8; ++i)
    score_step(s, ka, st.q[i], i);
}

// The softmax of one tile whose scores are s; keys k0 + key >= end are masked (only an item's
// last tile reaches past it). first: the wave's first tile of the item.
__device__ __attribute__((always_inline)) inline void wave_softmax(
    TileSoftmax& sm, WaveTileState& st, const f32x4 (&s)[2], unsigned k0, unsigned end,
    bool first, unsigned lane, const TileLane& tln) {
  if (k0 + kTileKeys > end)  // uniform
    tile_scores_joined<true>(sm, s, st.m, k0, end, lane, tln);
  else
    tile_scores_joined<false>(sm, s, st.m, k0, end, lane, tln);
  const bool moved = tile_decide(sm, st, first, tln);
  if (moved)
    tile_rescale(sm, st, first, tln);
  st.l += sm.lt;
}

// O += V^T P^T of one tile.
__device__ __attribute__((always_inline)) inline void wave_pv(WaveTileState& st,
                                                             const TileSoftmax& sm,
                                                             const cdna4::half8_t (&va)[16]) {
#pragma unroll
  for (int b = 0; b < 16; ++b)
    st.o[b] = mfma16(va[b], sm.pb, st.o[b]);
}

// The wave's state relative to its own true max: joined O (valid in lanes c < 8: head c,
// dimensions 16 b + 4 g + i) times o_scale (a power of two: the scale O is kept relative to, 1
// over f16 rows), l summed over the column (every lane), mt. A wave without tiles (any = false)
// gives mt = -inf, l = 0, O = 0.
struct WaveResult {
  float mt, l;
  f32x4 o[16];
};
__device__ __attribute__((always_inline)) inline void wave_result(WaveResult& r,
                                                                 const WaveTileState& st, bool any,
                                                                 float o_scale = 1.0f) {
  const float f = any ? __builtin_amdgcn_exp2f(st.m - st.mt) : 0.0f;
  const float fo = f * o_scale;
  r.mt = st.mt;
  r.l = cdna4::sum_xor32(cdna4::sum_xor16(st.l)) * f;
#pragma unroll
  for (unsigned b = 0; b < 16; ++b)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = st.o[b][i] * fo;
      r.o[b][i] = __builtin_fmaf(cdna4::dpp_mov<cdna4::kRowRor8>(x), kLoWeight, x);
    }
}

// The merge of the four wave results of one head: M = the largest true max, e_w = 2^(mt_w - M)
// (0 for a wave without keys; all e 0 when no wave has any), L = sum e_w l_w and O = sum e_w O_w,
// summed over w = 0 .. 3 in order.
struct WaveMergeScale {
  float e[4];
  float m, l;
};
__device__ __attribute__((always_inline)) inline WaveMergeScale wave_merge_scale(
    const float (&mt)[4], const float (&l)[4]) {
  WaveMergeScale ms;
  const float M = fmaxf(fmaxf(mt[0], mt[1]), fmaxf(mt[2], mt[3]));
  const bool none = M == -__builtin_inff();
  float L = 0.0f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    ms.e[w] = none ? 0.0f : __builtin_amdgcn_exp2f(mt[w] - M);
    L = __builtin_fmaf(ms.e[w], l[w], L);
  }
  ms.m = M;
  ms.l = L;
  return ms;
}
__device__ __attribute__((always_inline)) inline float4 wave_merge_o(const WaveMergeScale& ms,
                                                                    const float4 (&o)[4]) {
  float4 acc{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    acc.x = __builtin_fmaf(ms.e[w], o[w].x, acc.x);
    acc.y = __builtin_fmaf(ms.e[w], o[w].y, acc.y);
    acc.z = __builtin_fmaf(ms.e[w], o[w].z, acc.z);
    acc.w = __builtin_fmaf(ms.e[w], o[w].w, acc.w);
  }
  return acc;
}

// The exchange of wave results in LDS. O: wave w's chunk d (dimensions 4 d .. 4 d + 3, counted
// from the area's first block) of head h at float 4 (8 d + h) of its area; mt[8] and l[8] in its
// ml area. Lanes c < 8 store (consecutive heads in consecutive 16 bytes: no bank conflict).
__device__ __attribute__((always_inline)) inline void wave_merge_store(float* area_w, float* ml_w,
                                                                      const WaveResult& r,
                                                                      unsigned lane, unsigned b0,
                                                                      unsigned nb) {
  const unsigned g = lane >> 4, c = lane & 15u;
  if (c < 8) {
#pragma unroll
    for (unsigned b = 0; b < 16; ++b)
      if (b >= b0 && b < b0 + nb)
        *reinterpret_cast<float4*>(area_w + 4 * (8 * (4 * (b - b0) + g) + c)) =
            float4{r.o[b][0], r.o[b][1], r.o[b][2], r.o[b][3]};
    if (ml_w != nullptr && g == 0) {
      ml_w[c] = r.mt;
      ml_w[8 + c] = r.l;
    }
  }
}

// Head h's merge scale from the four ml areas (ml + w * ml_stride).
__device__ __attribute__((always_inline)) inline WaveMergeScale wave_merge_load_scale(
    const float* ml, unsigned ml_stride, unsigned h) {
  float mt[4], l[4];
#pragma unroll
  for (unsigned w = 0; w < 4; ++w) {
    mt[w] = ml[w * ml_stride + h];
    l[w] = ml[w * ml_stride + 8 + h];
  }
  return wave_merge_scale(mt, l);
}

// Merged chunk d of head h (area chunk index d, dimensions 4 dim_chunk ..) written to the partial.
__device__ __attribute__((always_inline)) inline void wave_merge_out(
    const float* area, unsigned stride, const WaveMergeScale& ms, unsigned d, unsigned dim_chunk,
    unsigned h, float* part_o, std::size_t base) {
  float4 o[4];
#pragma unroll
  for (unsigned w = 0; w < 4; ++w)
    o[w] = *reinterpret_cast<const float4*>(area + w * stride + 4 * (8 * d + h));
  *reinterpret_cast<float4*>(part_o + (base * kGroup + h) * attn::kDim + 4 * dim_chunk) =
      wave_merge_o(ms, o);
}

__device__ __attribute__((always_inline)) inline void wave_merge_ml_out(const WaveMergeScale& ms,
                                                                       unsigned h, float* part_m,
                                                                       float* part_l,
                                                                       std::size_t base) {
  part_m[base * kGroup + h] = ms.m * kLn2;  // -inf stays -inf for an empty item
  part_l[base * kGroup + h] = ms.l;
}

// Partial (m, l, o) of KV head kvh over keys [span.begin, span.end) at `base`, as
// split_partial_tiles computes it, with per-wave tiles: wave w takes tiles w, w + 4, ... and the
// four results merge at the end through the K slots (wave w's result in its own slot, which no
// other wave reads before the merge barrier). `more`: the workgroup runs another item
// afterwards (its LDS is then reused).
template <class Tiles>
__device__ __attribute__((always_inline)) inline void split_partial_waves(
    const float* __restrict__ q, const Tiles& tl, AttnSpan span, unsigned kvh, float* part_m,
    float* part_l, float* part_o, std::size_t base, TileShared& sh, bool more) {
  using cdna4::half8_t;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned n_tiles = (span.end - span.begin + kTileKeys - 1) / kTileKeys;
  const unsigned last_row = span.end - 1;  // unused when n_tiles == 0
  const unsigned nw = n_tiles > wave ? (n_tiles - wave + 3) / 4 : 0;  // this wave's tiles
  const unsigned k_lds = cdna4::lds_offset(sh.k[wave]), v_lds = cdna4::lds_offset(sh.v[wave]);
  const WaveCopy cp = wave_copy_offsets(lane);
  auto issue_k = [&](unsigned ti) __attribute__((always_inline)) {
    issue_wave_tile<false>(tl, span.begin + ti * kTileKeys, last_row, k_lds, cp, lane);
  };
  auto issue_v = [&](unsigned ti) __attribute__((always_inline)) {
    issue_wave_tile<true>(tl, span.begin + ti * kTileKeys, last_row, v_lds, cp, lane);
  };

  // The KV head's 8 query rows (wave w: rows 2 w, 2 w + 1), then the wave's first tile.
#pragma unroll
  for (unsigned i = 0; i < 2; ++i) {
    const unsigned h = 2 * wave + i;
    cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                      cdna4::lds_offset(sh.q[h]));
  }
  if (nw > 0) {
    issue_k(wave);
    issue_v(wave);
    cdna4::wait_vmcnt<16>();  // the queries and K landed; V may be in flight
  } else {
    cdna4::wait_vmcnt<0>();
  }
  tile_barrier();
  const TileLane tln = tile_lane(lane);
  const WaveOperands op = wave_operands(lane);
  WaveTileState st;
  wave_start(st, sh.q, lane, tln);

  // Tile j of the wave (tile ti = w + 4 j): its K landed. Once the K operands are in registers the
  // next tile's K goes into the slot, once the V operands are, its V. In flight after K of tile
  // ti: V of tile ti; after V of tile ti: K of the next tile.
  for (unsigned j = 0; j < nw; ++j) {
    const unsigned ti = wave + 4 * j;
    const bool next = j + 1 < nw;
    half8_t ka[2][8];
    read_k(ka, k_lds + op.kl);
    __builtin_amdgcn_sched_barrier(0);  // every K read in flight before the MFMAs
    f32x4 s[2];
    wave_scores(s, ka, st);
    if (next) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the K operands are in registers
      issue_k(ti + 4);
      cdna4::wait_vmcnt<16>();  // V of tile ti
    } else {
      cdna4::wait_vmcnt<0>();
    }
    half8_t va[16];
    read_v_all(va, v_lds, op.vl);
    __builtin_amdgcn_sched_barrier(0);  // the V reads in flight under the softmax
    TileSoftmax sm;
    wave_softmax(sm, st, s, span.begin + ti * kTileKeys, span.end, j == 0, lane, tln);
    if (next) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the V operands are in registers
      issue_v(ti + 4);
    }
    wave_pv(st, sm, va);
    if (next)
      cdna4::wait_vmcnt<16>();  // K of the next tile
  }

  // The merge through the K slots: wave w's result in its own slot (O in the first 8 KiB, mt and
  // l after it), which only it has used.
  {
    WaveResult r;
    wave_result(r, st, nw > 0);
    float* mine = reinterpret_cast<float*>(sh.k[wave]);
    wave_merge_store(mine, mine + 8 * attn::kDim, r, lane, 0, 16);
  }
  tile_barrier();
  {
    constexpr unsigned kStride = kTileBytes / 4;  // floats from one K slot to the next
    const float* area = reinterpret_cast<const float*>(sh.k[0]);
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

// PagedTiles of a split: the pages of its rows [span.begin, span.end), one per lane (at most 64
// pages; further ones are read from the table at use). The page-table slice is waited for here,
// before any tile copy is in flight.
__device__ __attribute__((always_inline)) inline PagedTiles paged_tiles(const PagedRows& rows,
                                                                        AttnSpan span) {
  const unsigned lane = threadIdx.x & 63u;
  const unsigned page0 = span.begin >> rows.log2_page;
  const unsigned npages =
      span.end > span.begin ? ((span.end - 1) >> rows.log2_page) - page0 + 1 : 0;
  int tab = lane < npages ? rows.table[page0 + lane] : 0;
  asm volatile("" : "+v"(tab));  // the load completes before the copies are issued
  return PagedTiles{rows, tab, page0};
}

}  // namespace decode_detail

namespace decode_detail {

// Items [first, first + count) of a split launch, item = kvh * n_splits + split (grid-stride, as
// the reference), in the given arithmetic.
template <DecodeArith kArith>
__device__ __attribute__((always_inline)) inline void split_items(const AttnSplitParams& p,
                                                                  unsigned first,
                                                                  unsigned count) {
  static_assert(kAttnSubChunk == SplitShared::kWaveCount * kAttnDecodeUnit,
                "a sub-chunk is one unit per wave");
  __shared__ SplitShared sh;
  for (unsigned item = first + blockIdx.y * gridDim.x + blockIdx.x; item < first + count;
       item += gridDim.x * gridDim.y) {
    const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
    const attn::half_t* K = p.k_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
    const attn::half_t* V = p.v_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
    split_partial<kArith>(p.q, K, V, p.len, attn_split_span(p.len, p.n_splits, split),
                          kAttnSubChunk, kvh, p.part_m, p.part_l, p.part_o,
                          std::size_t{kvh} * p.n_splits + split, sh,
                          item + gridDim.x * gridDim.y < first + count);
  }
}

}  // namespace decode_detail

namespace decode_detail {

// Splits longer than this many keys (8 tiles, two per wave) run with per-wave tiles.
constexpr unsigned kSplitWavesMinKeys = 8 * kTileKeys;

// Items [first, first + count) of a split launch on the matrix cores (split_partial_waves, or
// split_partial_tiles for short splits).
__device__ __attribute__((always_inline)) inline void split_items_mfma(const AttnSplitParams& p,
                                                                       unsigned first,
                                                                       unsigned count) {
  __shared__ TileShared sh;
  for (unsigned item = first + blockIdx.y * gridDim.x + blockIdx.x; item < first + count;
       item += gridDim.x * gridDim.y) {
    const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
    const std::size_t head = std::size_t{kvh} * p.max_ctx * attn::kDim;
    const AttnSpan span = attn_split_span(p.len, p.n_splits, split);
    const LinearTiles tl{p.k_cache + head, p.v_cache + head};
    const std::size_t base = std::size_t{kvh} * p.n_splits + split;
    const bool more = item + gridDim.x * gridDim.y < first + count;
    // Per-wave tiles once every wave has more than two of them; a shorter split keeps the
    // shared ring, whose first three tiles are in flight together (per-wave tiles would wait
    // for two load latencies one after the other).
    if (span.end - span.begin > kSplitWavesMinKeys)
      split_partial_waves(p.q, tl, span, kvh, p.part_m, p.part_l, p.part_o, base, sh, more);
    else
      split_partial_tiles(p.q, tl, span, kvh, p.part_m, p.part_l, p.part_o, base, sh, more);
  }
}

}  // namespace decode_detail

// Split-K flash decoding in the reference's precision (kernels/attention_decode.hpp:150-221: f32
// query, f32 scores and numerators, f32 accumulation over f16 K/V) on the matrix cores: each
// f32 operand is an exact f16 (hi, lo) pair, and the 8 heads x (hi, lo) fill the 16 columns of
// v_mfma_f32_16x16x32_f16 (split_partial_tiles). The KV cache streams through a 4-stage LDS ring
// of 32-key tiles; the max/sum reductions are DPP and lane-crossbar moves. Output: the
// reference's partial layout, m in natural-log units.
template <int kBlock>
__device__ void attn_split_op(const AttnSplitParams& p, unsigned first, unsigned count) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  decode_detail::split_items_mfma(p, first, count);
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1))) attn_split_kernel(AttnSplitParams p) {
  attn_split_op<kBlock>(p, 0, attn::kKvHeads * p.n_splits);
}

// The same split and arithmetic on wave64 VALU (no reference counterpart; same launch shape and
// partial layout). Each split's keys are streamed in 8-row units through per-wave LDS rings;
// scores are v_fma_mix_f32 products of the lane's f32 query slice and f16 K, summed by a
// DPP/crossbar reduce-scatter; P V is v_fma_mix_f32 of f32 numerators and f16 V: 512 products per
// key and head, one per instruction, which on MI355X is most of the HBM time of the same bytes.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_split_valu_kernel(AttnSplitParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  decode_detail::split_items<decode_detail::DecodeArith::kF32>(p, 0, attn::kKvHeads * p.n_splits);
}

// The same split with an f16 query and f16 numerators through v_dot2_f32_f16 (two products per
// instruction): half the VALU work of attn_split_kernel, per-head rel-L2 ~3e-4 against the FP64
// reference instead of ~1e-6 (no reference counterpart; same launch shape and partial layout).
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_split_f16q_kernel(AttnSplitParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  decode_detail::split_items<decode_detail::DecodeArith::kF16Query>(p, 0,
                                                                    attn::kKvHeads * p.n_splits);
}

// ------------------------------------------------------------------------------------------------
// Combine: LSE merge x sigmoid gate (reference: kernels/attention_decode.hpp:238-309)
// ------------------------------------------------------------------------------------------------

struct AttnCombineParams {
  const float* part_m;
  const float* part_l;
  const float* part_o;
  const float* qg;  // [16][512], for the gate half
  float* core;      // [16][256] = softmax(q K^T / 16) V * sigmoid(gate)
  unsigned n_splits;
};

namespace decode_detail {

// The merge of one head over one 64-dimension tile, computed by a full wave (lane = dimension).
// The result follows the reference's frozen FP32 order exactly: M = max_c m_c; for c in split
// order w = __expf(m_c - M), L = fma(w, l_c, L), o = fma(w, o_c, o); core = o / L / (1 + __expf(
// -gate)). Split statistics are per head, hence the same for the whole wave: lane c of a chunk
// loads m_c, l_c and forms w_c (a max is order-free and w_c depends only on m_c and M), and the
// wave publishes (w_c, l_c) through LDS. The tile's partial rows of a chunk of up to 128 splits
// (256 bytes each) are fetched with 16-byte loads -- lane l of load i takes split 4 i + l / 16,
// dimensions 4 (l % 16) .. + 3 -- all issued at once (32 loads per lane, under the 63
// outstanding loads a wave may have), and transposed through LDS, so a chunk costs one memory
// round trip; every lane then runs the ordered FMA chains over its dimension. Chunk entries past
// the last split are padded with w = l = 0 and a clamped, finite o: fma(0, x, acc) == acc
// exactly, so the padding cannot change a bit. Every template variant and the batched paths use
// this routine, so all are bit-identical to one another and to a one-thread-per-dimension serial
// loop.
constexpr unsigned kCombineChunk = 128;

struct CombineLds {
  float w[kCombineChunk], l[kCombineChunk];
  float o[kCombineChunk][cdna4::kLanes];  // [split of the chunk][dimension of the tile]
};

// One chunk of splits [base, base + nc), nc <= 4 kLoads, staged with kLoads 16-byte loads per
// lane and merged into (L, o). M is computed from the first chunk's statistics (and, past 128
// splits, the rest) when base == 0.
template <unsigned kLoads>
__device__ __attribute__((always_inline)) inline void combine_chunk(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ po_tile,
    unsigned n_splits, unsigned base, float& M, float& L, float& o, CombineLds& lds) {
  constexpr unsigned kStride = kGroup;  // partial rows per split
  constexpr std::size_t kOStride = std::size_t{kStride} * attn::kDim;
  const unsigned lane = cdna4::lane_id(), sub = lane >> 4, col = 4 * (lane & 15u);
  const unsigned last = n_splits - 1;
  float4 r[kLoads];
#pragma unroll
  for (unsigned i = 0; i < kLoads; ++i) {
    const unsigned c = base + 4 * i + sub;
    r[i] = *reinterpret_cast<const float4*>(po_tile + (c < last ? c : last) * kOStride + col);
  }
  constexpr unsigned kStat = kLoads * 4 > cdna4::kLanes ? 2 : 1;  // statistics per lane
  float mv[kStat], lv[kStat];
#pragma unroll
  for (unsigned j = 0; j < kStat; ++j) {
    const unsigned c = base + cdna4::kLanes * j + lane;
    mv[j] = c < n_splits ? pm[c * kStride] : -__builtin_inff();
    lv[j] = c < n_splits ? pl[c * kStride] : 0.0f;
  }
  if (base == 0) {
    M = mv[0];
#pragma unroll
    for (unsigned j = 1; j < kStat; ++j)
      M = fmaxf(M, mv[j]);
    for (unsigned c = kCombineChunk + lane; c < n_splits; c += cdna4::kLanes)  // > 128 splits
      M = fmaxf(M, pm[c * kStride]);
    M = cdna4::wave_allmax(M);
  }
#pragma unroll
  for (unsigned j = 0; j < kStat; ++j) {
    const unsigned c = cdna4::kLanes * j + lane;
    if (c < 4 * kLoads) {
      lds.w[c] = base + c < n_splits ? __expf(mv[j] - M) : 0.0f;
      lds.l[c] = lv[j];
    }
  }
#pragma unroll
  for (unsigned i = 0; i < kLoads; ++i)
    *reinterpret_cast<float4*>(&lds.o[4 * i + sub][col]) = r[i];
  __builtin_amdgcn_wave_barrier();
  // Every LDS value of the chunk into registers first (the reads pipeline), then the two ordered
  // chains from registers. Entries past the last split have w = l = 0 and a finite o.
  constexpr unsigned kN = 4 * kLoads;
  float ov[kN], wv[kN], lw[kN];
#pragma unroll
  for (unsigned c = 0; c < kN; c += 4) {
    const float4 w4 = *reinterpret_cast<const float4*>(&lds.w[c]);
    const float4 l4 = *reinterpret_cast<const float4*>(&lds.l[c]);
    wv[c] = w4.x, wv[c + 1] = w4.y, wv[c + 2] = w4.z, wv[c + 3] = w4.w;
    lw[c] = l4.x, lw[c + 1] = l4.y, lw[c + 2] = l4.z, lw[c + 3] = l4.w;
  }
#pragma unroll
  for (unsigned c = 0; c < kN; ++c)
    ov[c] = lds.o[c][lane];
#pragma unroll
  for (unsigned c = 0; c < kN; ++c) {
    L = __builtin_fmaf(wv[c], lw[c], L);
    o = __builtin_fmaf(wv[c], ov[c], o);
  }
  __builtin_amdgcn_wave_barrier();  // the next chunk (or merge) overwrites the LDS
}

// po_tile points at dimension 0 of the tile in split 0's row of the head (16-byte aligned); pm /
// pl at split 0's statistics; consecutive splits are kGroup rows apart.
__device__ __attribute__((always_inline)) inline float combine_wave(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ po_tile,
    unsigned n_splits, float gate, CombineLds& lds) {
  float L = 0.0f, o = 0.0f, M = -__builtin_inff();
  if (n_splits <= 16) {
    combine_chunk<4>(pm, pl, po_tile, n_splits, 0, M, L, o, lds);
  } else if (n_splits <= 32) {
    combine_chunk<8>(pm, pl, po_tile, n_splits, 0, M, L, o, lds);
  } else if (n_splits <= 64) {
    combine_chunk<16>(pm, pl, po_tile, n_splits, 0, M, L, o, lds);
  } else {
    for (unsigned base = 0; base < n_splits; base += kCombineChunk)
      combine_chunk<kCombineChunk / 4>(pm, pl, po_tile, n_splits, base, M, L, o, lds);
  }
  return o / L / (1.0f + __expf(-gate));
}

}  // namespace decode_detail

// Head/dimension tiles [first, first + count): item = h * (256 / kBlock) + tile, thread owns
// dimension tile * kBlock + threadIdx.x (grid-stride, as the reference). The template parameters
// and their constraints are the reference's; all variants share one arithmetic sequence.
template <int kBlock, bool kPrepared = false, int kPipeline = 1>
__device__ void attn_combine_op(const AttnCombineParams& p, unsigned first, unsigned count) {
  using namespace attn;
  constexpr int kGroup = kQHeads / kKvHeads, kTiles = kDim / kBlock;
  static_assert(kBlock % cdna4::kLanes == 0 && kDim % kBlock == 0);
  static_assert(!kPrepared || kBlock == cdna4::kLanes);
  static_assert(kPipeline == 1 || (kPrepared && kPipeline == 4));
  __shared__ decode_detail::CombineLds lds[kBlock / cdna4::kLanes];
  const unsigned wave = threadIdx.x / cdna4::kLanes;
  for (unsigned item = first + blockIdx.x; item < first + count; item += gridDim.x) {
    const unsigned h = item / kTiles, d0 = (item % kTiles) * kBlock + cdna4::kLanes * wave;
    const unsigned d = d0 + cdna4::lane_id();
    const unsigned kvh = h / kGroup, hl = h % kGroup;
    const std::size_t i0 = std::size_t{kvh} * p.n_splits * kGroup + hl;
    p.core[h * kDim + d] = decode_detail::combine_wave(
        p.part_m + i0, p.part_l + i0, p.part_o + i0 * kDim + d0, p.n_splits,
        p.qg[h * 2 * kDim + kDim + d], lds[wave]);
  }
}

template <int kBlock, bool kPrepared = false, int kPipeline = 1>
__global__ void __launch_bounds__(kBlock) attn_combine_kernel(AttnCombineParams p) {
  attn_combine_op<kBlock, kPrepared, kPipeline>(p, 0, attn::kQHeads * (attn::kDim / kBlock));
}

// ------------------------------------------------------------------------------------------------
// Single-launch decode (no reference counterpart: the reference launches the split and then the
// combine, src/engine/attention.hip:103-109). Grid (n_splits, 2) x 256, exactly one item per
// workgroup. Each workgroup computes its split's partial as attn_split_kernel does, stores it
// agent-coherently, waits for the stores, and takes a ticket from its KV head's arrival counter.
// The last T = min(n_splits, 32) arrivals of a KV head become its mergers: merger j waits until
// every split of the head has arrived (only the stragglers remain by then), then merges tiles
// j, j + T, ... of the head's 32 (head, 64-dimension) tiles and applies the gate. Earlier arrivals
// exit at once, so at most 2 T workgroups ever wait, and every workgroup still to start finds a
// free CU as long as the device has more CUs than that (the host checks it). The wait is bounded
// (kFusedSpinTicks); a merger that gives up writes NaN to its tiles instead of hanging. The last
// merger to finish resets the head's counters: every launch leaves them zero, and launches that
// overlap on one `sync` buffer race.
//
// Merge order (fixed, so results are bit-equal from call to call): M = max_c m_c; w_c =
// __expf(m_c - M); wave w of the merger sums w_c o_c over its quarter of the splits in split
// order; o = ((S_0 + S_1) + S_2) + S_3; L = the wave-reduction of w_c l_c; core = o / L /
// (1 + __expf(-gate)). Not the frozen order of attn_combine_kernel, and within the reference's
// rel-L2 gate of it.
// ------------------------------------------------------------------------------------------------

struct AttnDecodeFusedParams {
  AttnSplitParams s;
  const float* qg;  // [16][512]: gate at h * 512 + 256 + d
  float* core;      // [16][256]
  unsigned* sync;   // [2 KV heads][2]: arrivals, finished mergers; zero before the first launch
};

constexpr unsigned kFusedMaxMergers = 32;  // per KV head: one per (head, 64-dimension) tile
constexpr unsigned long long kFusedSpinTicks = 5000000;  // 50 ms of the 100 MHz s_memrealtime

__host__ __device__ constexpr unsigned attn_fused_mergers(unsigned n_splits) {
  return n_splits < kFusedMaxMergers ? n_splits : kFusedMaxMergers;
}

namespace decode_detail {

struct FusedMergeLds {
  float w[kAttnTargetSplits], l[kAttnTargetSplits];
  float part[4][cdna4::kLanes];
  float red[4];
};

// Tile t of KV head kvh (head 8 kvh + t / 4, dimensions 64 (t % 4) .. + 63) from the n partials.
__device__ __attribute__((always_inline)) inline void fused_merge_tile(
    const AttnDecodeFusedParams& p, unsigned kvh, unsigned t, bool ok, FusedMergeLds& lds) {
  const unsigned n = p.s.n_splits, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const unsigned hl = t / 4, d = 64 * (t % 4) + lane;
  const std::size_t i0 = std::size_t{kvh} * n * kGroup + hl;  // split c's statistics: i0 + 8 c
  const unsigned part_floats = 2 * n * kGroup * attn::kDim;
  const auto o_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.s.part_o), 0,
                                                        static_cast<int>(4 * part_floats),
                                                        0x00020000);
  // This wave's splits [c0, c1): all its partial values in flight at once (at most 32).
  const unsigned per = (n + 3) / 4, c0 = wave * per, c1 = c0 + per < n ? c0 + per : n;
  float ov[32];
#pragma unroll
  for (unsigned i = 0; i < 32; ++i) {
    const unsigned c = c0 + i;
    ov[i] = c < c1 ? __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                   o_rsrc,
                                                   static_cast<int>(4 * ((i0 + std::size_t{c} *
                                                                                   kGroup) *
                                                                              attn::kDim + d)),
                                                   0, kSc1))
                   : 0.0f;
  }
  float mv = -__builtin_inff(), lv = 0.0f;
  if (tid < n) {
    mv = __hip_atomic_load(p.s.part_m + i0 + std::size_t{tid} * kGroup, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    lv = __hip_atomic_load(p.s.part_l + i0 + std::size_t{tid} * kGroup, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
  const float wm = cdna4::wave_allmax(mv);
  if (lane == 0)
    lds.red[wave] = wm;
  __syncthreads();
  const float M = fmaxf(fmaxf(lds.red[0], lds.red[1]), fmaxf(lds.red[2], lds.red[3]));
  const float wc = tid < n ? __expf(mv - M) : 0.0f;
  if (tid < n)
    lds.w[tid] = wc, lds.l[tid] = lv;
  __syncthreads();  // every weight published; lds.red is read
  const float wl = cdna4::wave_allsum(wc * lv);
  float acc = 0.0f;
#pragma unroll
  for (unsigned i = 0; i < 32; ++i)
    if (c0 + i < c1)
      acc = __builtin_fmaf(lds.w[c0 + i], ov[i], acc);
  lds.part[wave][lane] = acc;
  if (lane == 0)
    lds.red[wave] = wl;
  __syncthreads();
  if (wave == 0) {
    const float o = ((lds.part[0][lane] + lds.part[1][lane]) + lds.part[2][lane]) +
                    lds.part[3][lane];
    const float L = ((lds.red[0] + lds.red[1]) + lds.red[2]) + lds.red[3];
    const unsigned h = kvh * kGroup + hl;
    const float gate = p.qg[h * 2 * attn::kDim + attn::kDim + d];
    p.core[h * attn::kDim + d] = ok ? o / L / (1.0f + __expf(-gate)) : __builtin_nanf("");
  }
  __syncthreads();  // the LDS is reused by the next tile
}

}  // namespace decode_detail

template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_decode_fused_kernel(AttnDecodeFusedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  using namespace decode_detail;
  __shared__ TileShared sh;
  const unsigned n = p.s.n_splits;
  const unsigned kvh = blockIdx.y, split = blockIdx.x;  // grid (n_splits, 2)
  const std::size_t head = std::size_t{kvh} * p.s.max_ctx * attn::kDim;
  split_partial_tiles<LinearTiles, true>(
      p.s.q, LinearTiles{p.s.k_cache + head, p.s.v_cache + head},
      attn_split_span(p.s.len, n, split), kvh, p.s.part_m, p.s.part_l, p.s.part_o,
      std::size_t{kvh} * n + split, sh, false, 2 * n * kGroup * attn::kDim);
  // Arrival: this workgroup's partial stores complete (each wave), then one ticket.
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0) expcnt(0) lgkmcnt(0)
  __syncthreads();
  auto* lds = reinterpret_cast<FusedMergeLds*>(&sh);
  auto* flag = reinterpret_cast<unsigned*>(&lds->red[0]);
  unsigned* const arrivals = p.sync + 2 * kvh;
  unsigned* const finished = arrivals + 1;
  if (threadIdx.x == 0)
    *flag = __hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  const unsigned ticket = *flag, mergers = attn_fused_mergers(n);
  if (ticket + mergers < n)  // uniform
    return;
  const unsigned j = ticket + mergers - n;
  __syncthreads();  // the ticket is read before the flag is reused
  if (threadIdx.x == 0) {  // every split of this KV head has arrived (bounded wait)
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    unsigned ok = 1;
    while (__hip_atomic_load(arrivals, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < n) {
      if (__builtin_amdgcn_s_memrealtime() - t0 > kFusedSpinTicks) {
        ok = 0;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    *flag = ok;
  }
  __syncthreads();
  const bool ok = *flag != 0;
  __syncthreads();
  for (unsigned t = j; t < kGroup * 4; t += mergers)
    fused_merge_tile(p, kvh, t, ok, *lds);
  if (threadIdx.x == 0) {
    const unsigned done = __hip_atomic_fetch_add(finished, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    if (done + 1 == mergers) {  // every merger has passed its wait: reset for the next launch
      __hip_atomic_store(arrivals, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(finished, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Ragged batched decode (no reference counterpart: the reference is batch-1). Semantics per
// sequence = split + combine above, with a dense gate tensor.
// ------------------------------------------------------------------------------------------------

// Keys per split for the batched path: large enough that the partials stay a few percent of the
// KV bytes, small enough that a batch of long and short sequences balances across CUs. The partial
// buffers are sized for this chunk; a launch may split at kAttnRaggedWideChunk instead
// (attn_ragged_chunk), which needs fewer partials.
constexpr unsigned kAttnRaggedChunk = 512;
constexpr unsigned kAttnRaggedWideChunk = 1024;

// The chunk a launch splits at: the wide one when even that gives at least four items per CU
// for a batch of `batch` sequences of up to max_len keys (fewer per-item merges in the streaming
// kernel; measured on C5, 64 sequences: 211 us against 230 us), else kAttnRaggedChunk so that
// small batches still fill the CUs. cus = 0 (unknown) keeps kAttnRaggedChunk.
__host__ __device__ constexpr unsigned attn_ragged_chunk(unsigned batch, unsigned max_len,
                                                        unsigned cus) {
  const unsigned long long items = 2ull * batch *
                                   ((max_len + kAttnRaggedWideChunk - 1) / kAttnRaggedWideChunk);
  return cus > 0 && items >= 4ull * cus ? kAttnRaggedWideChunk : kAttnRaggedChunk;
}

__host__ __device__ constexpr unsigned attn_ragged_splits(unsigned max_len) {
  const unsigned n = (max_len + kAttnRaggedChunk - 1) / kAttnRaggedChunk;
  return n == 0 ? 1 : n;
}

struct AttnRaggedParams {
  const float* q;               // [batch][16][256] (unscaled)
  const float* gate;            // [batch][16][256]
  const attn::half_t* k_cache;  // sequence s: K [2][lens[s]][256] at kv_offsets[s]
  const attn::half_t* v_cache;
  const uint64_t* kv_offsets;  // [batch], in halves (device)
  const uint32_t* lens;        // [batch] (device)
  float* core;                 // [batch][16][256]
  float* part_m;               // [batch][2][s_max][8]
  float* part_l;
  float* part_o;  // [batch][2][s_max][8][256]
  unsigned batch, s_max;
  unsigned len_cap;  // keys a sequence can hold (the paged layout's pages x page size); lens
                     // past it count as len_cap. ~0u for the contiguous ragged layout.
  unsigned chunk;    // keys per split (attn_ragged_chunk), the same in the split and the merge
};

// Splits of a sequence of len keys: one per `chunk` keys, at most s_max.
__host__ __device__ inline unsigned attn_ragged_seq_splits(unsigned len, unsigned s_max,
                                                           unsigned chunk) {
  const unsigned n = (len + chunk - 1) / chunk;
  return n < s_max ? n : s_max;
}

// One workgroup per (sequence, KV head, split slot); slots past the sequence's split count exit.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1))) attn_ragged_split_kernel(AttnRaggedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::TileShared sh;
  const unsigned item = blockIdx.x;
  const unsigned split = item % p.s_max, kvh = (item / p.s_max) % attn::kKvHeads;
  const unsigned seq = item / (p.s_max * attn::kKvHeads);
  if (seq >= p.batch)
    return;
  const unsigned len = p.lens[seq];
  const unsigned n_splits = attn_ragged_seq_splits(len, p.s_max, p.chunk);
  if (split >= n_splits)
    return;
  const std::size_t kv0 = p.kv_offsets[seq] + std::size_t{kvh} * len * attn::kDim;
  decode_detail::split_partial_waves(
      p.q + std::size_t{seq} * attn::kQHeads * attn::kDim,
      decode_detail::LinearTiles{p.k_cache + kv0, p.v_cache + kv0},
      attn_split_span(len, n_splits, split), kvh, p.part_m, p.part_l, p.part_o,
      (std::size_t{seq} * attn::kKvHeads + kvh) * p.s_max + split, sh, false);
}

// The same splits on one workgroup per CU (no reference counterpart). Each workgroup takes items
// w, w + G, w + 2 G, ... of the batch's (sequence, KV head, split) list (sequence-major, KV head,
// then split; each workgroup computes the list's sequence offsets itself), so the workgroups'
// item counts differ by at most one. Per item, wave v takes the item's tiles v, v + 4, ... as
// split_partial_waves does, and each wave's tile stream runs straight across item boundaries:
// its next tile, whichever item holds it, is issued as soon as the current one's operands are
// in registers. Each item's query rows go into one of two LDS slots while the previous item is
// processed. Per item the arithmetic, the partial and its layout are split_partial_waves' (so
// the partials equal attn_ragged_split_kernel's bit for bit), and attn_ragged_combine_kernel
// merges them. Batches of up to kRaggedStreamMaxBatch sequences whose per-workgroup item count
// fits kRaggedStreamMaxItems (attn_ragged_stream_fits): one item per lane of a wave.
constexpr unsigned kRaggedStreamMaxBatch = 512;
constexpr unsigned kRaggedStreamMaxItems = 64;

__host__ __device__ constexpr bool attn_ragged_stream_fits(unsigned batch, unsigned s_max,
                                                         unsigned grid) {
  return batch <= kRaggedStreamMaxBatch && grid > 0 &&
         (std::size_t{batch} * attn::kKvHeads * s_max + grid - 1) / grid <= kRaggedStreamMaxItems;
}

namespace decode_detail {

// 160 KiB: the four waves' K and V slots, two query-row slots, and the O exchange of one merge
// pass (128 dimensions of four wave results), which the set-up's sequence offsets use before.
struct alignas(1024) StreamShared {
  unsigned char k[4][kTileBytes];
  unsigned char v[4][kTileBytes];
  float q[2][kGroup][attn::kDim];
  float merge[4][32 * kGroup * 4];
};
static_assert(sizeof(StreamShared) == 160 * 1024, "the CU's LDS");
static_assert((kRaggedStreamMaxBatch + 1) * sizeof(unsigned) <= sizeof(StreamShared::merge),
              "sequence offsets in the merge area");

// The batch of a streaming launch, whatever its layout.
struct StreamBatch {
  const float* q;  // [batch][16][256] (unscaled)
  float* part_m;
  float* part_l;
  float* part_o;
  const uint32_t* lens;
  unsigned batch, s_max, len_cap, chunk;
};

__device__ __attribute__((always_inline)) inline unsigned lane_value(unsigned v, unsigned j) {
  return static_cast<unsigned>(
      __builtin_amdgcn_readlane(static_cast<int>(v), static_cast<int>(j)));
}

// Where an item's tiles lie. describe() runs in lane j for item j (its sequence, KV head and
// capped length); prepare(j, ...) runs, wave-uniform, for a tile before issue<kV>(j, ...) copies
// its K and V (the same tile, in that order).
struct RaggedStreamSource {  // contiguous rows: K [2][len][256] at kv_offsets[s]
  const attn::half_t* k_cache;
  const attn::half_t* v_cache;
  const uint64_t* kv_offsets;
  unsigned kv_lo = 0, kv_hi = 0;  // lane j: item j's element offset
  __device__ __attribute__((always_inline)) void describe(unsigned seq, unsigned kvh,
                                                          unsigned len) {
    const std::size_t kv0 = kv_offsets[seq] + std::size_t{kvh} * len * attn::kDim;
    kv_lo = static_cast<unsigned>(kv0);
    kv_hi = static_cast<unsigned>(kv0 >> 32);
  }
  __device__ __attribute__((always_inline)) void prepare(unsigned, unsigned, unsigned, unsigned,
                                                         unsigned) {}
  template <bool kV>
  __device__ __attribute__((always_inline)) void issue(unsigned j, unsigned k0, unsigned last_row,
                                                       unsigned lds, const WaveCopy& cp,
                                                       unsigned lane) const {
    const std::size_t kv0 = (std::size_t{lane_value(kv_hi, j)} << 32) | lane_value(kv_lo, j);
    issue_wave_tile<kV>(LinearTiles{k_cache + kv0, v_cache + kv0}, k0, last_row, lds, cp, lane);
  }
};

// The pages of one tile's four 8-row groups (a group never straddles pages: pages hold a
// multiple of 8 rows and spans start at multiples of 8; a group past the item's last row reads
// that row, in the page of the group holding it), read from the page table with scalar loads
// when the tile is prepared, one tile ahead of its copy.
struct PagedTileRows {
  const attn::half_t* k_pages;
  const attn::half_t* v_pages;
  std::size_t page_halves, head_off;
  unsigned log2_page;
  int page0, page1, page2, page3;  // group g's page (the group is a compile-time index below)
  template <unsigned G>
  __device__ __attribute__((always_inline)) std::size_t at(unsigned row) const {
    const int pg = G == 0 ? page0 : G == 1 ? page1 : G == 2 ? page2 : page3;
    return std::size_t(static_cast<unsigned>(pg)) * page_halves + head_off +
           std::size_t{row & ((1u << log2_page) - 1u)} * attn::kDim;
  }
};
template <bool kV, unsigned G>
__device__ __attribute__((always_inline)) inline const attn::half_t* tile_group_row(
    const PagedTileRows& tl, unsigned row) {
  return (kV ? tl.v_pages : tl.k_pages) + tl.template at<G>(row);
}

struct PagedStreamSource {
  const attn::half_t* k_pages;
  const attn::half_t* v_pages;
  const int32_t* page_table;  // [batch][max_pages]
  unsigned max_pages, log2_page;
  PagedTileRows next{};
  __device__ __attribute__((always_inline)) void describe(unsigned, unsigned, unsigned) {}
  // Tile at key k0 of item (seq, kvh) whose last row is last_row: the page of each group's first
  // row (or of last_row for groups past it), read through the constant address space so the
  // loads are scalar (the table is not written by the launch).
  __device__ __attribute__((always_inline)) void prepare(unsigned seq, unsigned kvh, unsigned k0,
                                                         unsigned last_row, unsigned) {
    typedef const __attribute__((address_space(4))) int32_t ctab;
    ctab* row = (ctab*)(page_table + std::size_t{seq} * max_pages);  // NOLINT: address space
    next.k_pages = k_pages;
    next.v_pages = v_pages;
    next.log2_page = log2_page;
    next.page_halves = std::size_t{2} * attn::kDim << log2_page;
    next.head_off = std::size_t{kvh} * attn::kDim << log2_page;
    auto page_of = [&](unsigned g) __attribute__((always_inline)) {
      const unsigned r = k0 + 8 * g < last_row ? k0 + 8 * g : last_row;
      return row[r >> log2_page];
    };
    next.page0 = page_of(0);
    next.page1 = page_of(1);
    next.page2 = page_of(2);
    next.page3 = page_of(3);
  }
  template <bool kV>
  __device__ __attribute__((always_inline)) void issue(unsigned, unsigned k0, unsigned last_row,
                                                       unsigned lds, const WaveCopy& cp,
                                                       unsigned lane) const {
    issue_wave_tile<kV>(next, k0, last_row, lds, cp, lane);
  }
};

// The streaming split over the batch's items (attn_ragged_stream_kernel's description), with
// the tiles where Src says they are.
template <class Src>
__device__ __attribute__((always_inline)) inline void stream_items(const StreamBatch& p, Src& src,
                                                                  StreamShared& sh) {
  using cdna4::half8_t;
  constexpr unsigned kBlock = 256;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned G = gridDim.x, w = blockIdx.x;
  unsigned* prefix = reinterpret_cast<unsigned*>(sh.merge);

  // Sequence offsets of the item list (wave 0: 64 sequences per step, an inclusive scan).
  if (wave == 0) {
    unsigned run = 0;
    if (lane == 0)
      prefix[0] = 0;
    for (unsigned base = 0; base < p.batch; base += cdna4::kLanes) {
      const unsigned s_ = base + lane;
      unsigned cnt = 0;
      if (s_ < p.batch) {
        const unsigned len = p.lens[s_] < p.len_cap ? p.lens[s_] : p.len_cap;
        cnt = attn::kKvHeads * attn_ragged_seq_splits(len, p.s_max, p.chunk);
      }
      unsigned incl = cnt;
#pragma unroll
      for (unsigned d = 1; d < cdna4::kLanes; d *= 2) {
        const unsigned up = __shfl_up(incl, d, cdna4::kLanes);
        incl += lane >= d ? up : 0u;
      }
      if (s_ < p.batch)
        prefix[s_ + 1] = run + incl;
      run += __shfl(incl, cdna4::kLanes - 1, cdna4::kLanes);
    }
  }
  __syncthreads();
  // Every wave holds the descriptors of the workgroup's items, item j in lane j: key span,
  // partial row group, tile count (0 for an empty span), sequence and KV head (and what Src
  // keeps).
  const unsigned total = prefix[p.batch];
  const unsigned n_items = w < total ? (total - w + G - 1) / G : 0;
  unsigned it_begin = 0, it_end = 0, it_part = 0, it_tiles = 0, it_seq = 0, it_kvh = 0;
  if (lane < n_items) {
    const unsigned k = w + lane * G;
    unsigned lo = 0, hi = p.batch;  // the sequence s with prefix[s] <= k < prefix[s + 1]
    while (hi - lo > 1) {
      const unsigned mid = (lo + hi) / 2;
      if (prefix[mid] <= k)
        lo = mid;
      else
        hi = mid;
    }
    const unsigned r = k - prefix[lo], n = (prefix[lo + 1] - prefix[lo]) / 2;
    const unsigned kvh = r / n, split = r % n;
    const unsigned len = p.lens[lo] < p.len_cap ? p.lens[lo] : p.len_cap;
    const AttnSpan span = attn_split_span(len, n, split);
    src.describe(lo, kvh, len);
    it_begin = span.begin;
    it_end = span.end;
    it_part = (lo * attn::kKvHeads + kvh) * p.s_max + split;
    it_tiles = (span.end - span.begin + kTileKeys - 1) / kTileKeys;
    it_seq = lo;
    it_kvh = kvh;
  }
  // Items with an empty span (capped split counts) have no tiles: their partial is written here,
  // (-inf, 0, 0) as the split writes it, and the item loop skips them.
  for (unsigned j = 0; j < n_items; ++j) {
    if (lane_value(it_tiles, j) != 0)
      continue;
    const unsigned part = lane_value(it_part, j);
    float* po = p.part_o + std::size_t{part} * kGroup * attn::kDim;
#pragma unroll
    for (unsigned i = 0; i < kGroup * attn::kDim / kBlock; ++i)
      po[i * kBlock + t] = 0.0f;
    if (t < kGroup) {
      p.part_m[std::size_t{part} * kGroup + t] = -__builtin_inff();
      p.part_l[std::size_t{part} * kGroup + t] = 0.0f;
    }
  }
  auto next_item = [&](unsigned j) __attribute__((always_inline)) {  // first non-empty >= j
    while (j < n_items && lane_value(it_tiles, j) == 0)
      ++j;
    return j;
  };
  // The first item from j on with more than `wave` tiles (n_items if none): where this wave's
  // next tile lies when the current item has no more of its tiles.
  auto wave_item = [&](unsigned j) __attribute__((always_inline)) {
    while (j < n_items && lane_value(it_tiles, j) <= wave)
      ++j;
    return j;
  };

  // Vector-memory instructions this wave has issued since the set-up, and the counts right after
  // the copies the waits below are for: each wait allows what was issued after its copy.
  unsigned issued = 0;
  const unsigned k_lds = cdna4::lds_offset(sh.k[wave]), v_lds = cdna4::lds_offset(sh.v[wave]);
  const WaveCopy cp = wave_copy_offsets(lane);
  auto prepare = [&](unsigned j, unsigned ti) __attribute__((always_inline)) {
    src.prepare(lane_value(it_seq, j), lane_value(it_kvh, j),
                lane_value(it_begin, j) + ti * kTileKeys, lane_value(it_end, j) - 1, j);
  };
  auto issue_k = [&](unsigned j, unsigned ti) __attribute__((always_inline)) {
    src.template issue<false>(j, lane_value(it_begin, j) + ti * kTileKeys,
                              lane_value(it_end, j) - 1, k_lds, cp, lane);
    issued += 16;
  };
  auto issue_v = [&](unsigned j, unsigned ti) __attribute__((always_inline)) {
    src.template issue<true>(j, lane_value(it_begin, j) + ti * kTileKeys,
                             lane_value(it_end, j) - 1, v_lds, cp, lane);
    issued += 16;
  };
  auto issue_q = [&](unsigned j, unsigned slot) __attribute__((always_inline)) {
    const float* q = p.q + std::size_t{lane_value(it_seq, j)} * attn::kQHeads * attn::kDim;
    const unsigned kvh = lane_value(it_kvh, j);
#pragma unroll
    for (unsigned i = 0; i < 2; ++i) {
      const unsigned h = 2 * wave + i;
      cdna4::lds_load16(q + (std::size_t{kvh} * kGroup + h) * attn::kDim + 4 * lane,
                        cdna4::lds_offset(sh.q[slot][h]));
    }
    issued += 2;
  };

  unsigned jc = next_item(0);  // the item being computed
  if (jc >= n_items)           // uniform
    return;
  issue_q(jc, 0);
  unsigned mark_q = issued;
  // The wave's tile cursor: item pj, tile pt (pj = n_items: none); the counts after its copies.
  unsigned pj = wave_item(jc), pt = wave, mark_k = 0, mark_v = 0;
  if (pj < n_items) {
    prepare(pj, pt);
    issue_k(pj, pt);
    mark_k = issued;
    issue_v(pj, pt);
    mark_v = issued;
  }
  const TileLane tln = tile_lane(lane);
  const WaveOperands op = wave_operands(lane);
  const unsigned h = t % 8, d = t / 8;  // the merge's head and dimension chunk
  WaveTileState st;
  for (unsigned ord = 0;; ++ord) {
    wait_vm_at_most(issued - mark_q);  // this wave's query rows of item jc
    tile_barrier();                    // every wave's
    wave_start(st, sh.q[ord & 1u], lane, tln);
    tile_barrier();  // every wave has read slot ord % 2 (its m, l exchange follows below)
    const unsigned jn = next_item(jc + 1);
    if (jn < n_items) {  // the next item's query rows into the other slot
      issue_q(jn, (ord + 1) & 1u);
      mark_q = issued;
    }
    const unsigned begin = lane_value(it_begin, jc), end = lane_value(it_end, jc);
    bool any = false;
    while (pj == jc) {
      const unsigned ti = pt, mk = mark_k, mv = mark_v;
      // The next tile of this wave: the item's tile ti + 4, else its first tile in a later item.
      unsigned nj = jc, nt = ti + 4;
      if (nt >= lane_value(it_tiles, jc)) {
        nj = wave_item(jc + 1);
        nt = wave;
      }
      const bool next = nj < n_items;
      if (next)
        prepare(nj, nt);
      wait_vm_at_most(issued - mk);  // K of tile ti
      half8_t ka[2][8];
      read_k(ka, k_lds + op.kl);
      __builtin_amdgcn_sched_barrier(0);
      f32x4 s[2];
      wave_scores(s, ka, st);
      if (next) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the K operands are in registers
        issue_k(nj, nt);
        mark_k = issued;
      }
      wait_vm_at_most(issued - mv);  // V of tile ti
      half8_t va[16];
      read_v_all(va, v_lds, op.vl);
      __builtin_amdgcn_sched_barrier(0);
      TileSoftmax sm;
      wave_softmax(sm, st, s, begin + ti * kTileKeys, end, !any, lane, tln);
      if (next) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the V operands are in registers
        issue_v(nj, nt);
        mark_v = issued;
      }
      wave_pv(st, sm, va);
      any = true;
      pj = nj;
      pt = nt;
    }
    // The item's partial: the four wave results merged in two passes of 128 dimensions through
    // sh.merge; mt and l through the query slot this item used (read by every wave above).
    {
      WaveResult r;
      wave_result(r, st, any);
      float* ml = &sh.q[ord & 1u][0][0];
      const std::size_t part = lane_value(it_part, jc);
      wave_merge_store(sh.merge[wave], ml + 16 * wave, r, lane, 0, 8);
      tile_barrier();
      const WaveMergeScale ms = wave_merge_load_scale(ml, 16, h);
      wave_merge_out(&sh.merge[0][0], 32 * kGroup * 4, ms, d, d, h, p.part_o, part);
      if (d == 0)
        wave_merge_ml_out(ms, h, p.part_m, p.part_l, part);
      tile_barrier();
      wave_merge_store(sh.merge[wave], nullptr, r, lane, 8, 8);
      tile_barrier();
      wave_merge_out(&sh.merge[0][0], 32 * kGroup * 4, ms, d, d + 32, h, p.part_o, part);
      issued += 2;  // at least one 16-byte store per pass and wave
    }
    jc = jn;
    if (jc >= n_items)
      break;
  }
}

}  // namespace decode_detail

template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_ragged_stream_kernel(AttnRaggedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::StreamShared sh;
  decode_detail::RaggedStreamSource src{p.k_cache, p.v_cache, p.kv_offsets};
  decode_detail::stream_items(
      decode_detail::StreamBatch{p.q, p.part_m, p.part_l, p.part_o, p.lens, p.batch, p.s_max,
                                 p.len_cap, p.chunk},
      src, sh);
}

// One 64-thread workgroup per (sequence, head, 64-dim tile); the merge is combine_wave's. (A
// template, so every translation unit including this header may instantiate it.)
template <int = 0>
__global__ void __launch_bounds__(64) attn_ragged_combine_kernel(AttnRaggedParams p) {
  constexpr unsigned kGroup = attn::kQHeads / attn::kKvHeads, kTiles = attn::kDim / 64;
  const unsigned item = blockIdx.x;
  const unsigned seq = item / (attn::kQHeads * kTiles), h = (item / kTiles) % attn::kQHeads;
  const unsigned d = (item % kTiles) * 64 + threadIdx.x;
  if (seq >= p.batch)
    return;
  const std::size_t out = (std::size_t{seq} * attn::kQHeads + h) * attn::kDim + d;
  const unsigned len = p.lens[seq] < p.len_cap ? p.lens[seq] : p.len_cap;
  const unsigned n_splits = attn_ragged_seq_splits(len, p.s_max, p.chunk);
  if (n_splits == 0) {
    p.core[out] = 0.0f;
    return;
  }
  const unsigned kvh = h / kGroup, hl = h % kGroup;
  const std::size_t i0 = (std::size_t{seq} * attn::kKvHeads + kvh) * p.s_max * kGroup + hl;
  __shared__ decode_detail::CombineLds lds;
  p.core[out] = decode_detail::combine_wave(p.part_m + i0, p.part_l + i0,
                                           p.part_o + i0 * attn::kDim + (d - threadIdx.x),
                                           n_splits, p.gate[out], lds);
}

// ------------------------------------------------------------------------------------------------
// Paged batched decode (no reference counterpart): the ragged decode over a pool of KV pages.
// Page id g holds [2 KV heads][page][256] f16 at g * 2 * page * 256 halves of k_pages / v_pages;
// sequence s's positions [j page, (j + 1) page) are in page page_table[s * max_pages + j]; a
// sequence attends to min(lens[s], max_pages x page) keys. Same splits, arithmetic and partial
// layout as the ragged path, so the outputs are bit-identical to it on the same keys;
// attn_ragged_combine_kernel (with that cap) merges the partials.
// ------------------------------------------------------------------------------------------------

struct AttnPagedParams {
  const float* q;                // [batch][16][256] (unscaled)
  const attn::half_t* k_pages;   // [pages][2][page][256]
  const attn::half_t* v_pages;
  const int32_t* page_table;     // [batch][max_pages] (device)
  const uint32_t* lens;          // [batch] (device)
  float* part_m;                 // [batch][2][s_max][8]
  float* part_l;
  float* part_o;                 // [batch][2][s_max][8][256]
  unsigned batch, s_max, max_pages, log2_page;
  unsigned chunk;                // keys per split (attn_ragged_chunk)
};

// Keys a paged sequence can hold: a longer lens[s] attends to its first max_pages pages only
// (its page-table row has no entries past them).
__host__ __device__ inline unsigned attn_paged_len_cap(unsigned max_pages, unsigned log2_page) {
  const unsigned long long cap = static_cast<unsigned long long>(max_pages) << log2_page;
  return cap < 0xFFFFFFFFull ? static_cast<unsigned>(cap) : 0xFFFFFFFFu;
}

// One workgroup per (sequence, KV head, split slot), as attn_ragged_split_kernel.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1))) attn_paged_split_kernel(AttnPagedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::TileShared sh;
  const unsigned item = blockIdx.x;
  const unsigned split = item % p.s_max, kvh = (item / p.s_max) % attn::kKvHeads;
  const unsigned seq = item / (p.s_max * attn::kKvHeads);
  if (seq >= p.batch)
    return;
  const unsigned cap = attn_paged_len_cap(p.max_pages, p.log2_page);
  const unsigned len = p.lens[seq] < cap ? p.lens[seq] : cap;
  const unsigned n_splits = attn_ragged_seq_splits(len, p.s_max, p.chunk);
  if (split >= n_splits)
    return;
  const decode_detail::PagedRows rows{
      p.k_pages, p.v_pages, p.page_table + std::size_t{seq} * p.max_pages, p.log2_page,
      std::size_t{2} * attn::kDim << p.log2_page,
      std::size_t{kvh} * attn::kDim << p.log2_page};
  const AttnSpan span = attn_split_span(len, n_splits, split);
  decode_detail::split_partial_waves(p.q + std::size_t{seq} * attn::kQHeads * attn::kDim,
                                     decode_detail::paged_tiles(rows, span), span, kvh, p.part_m,
                                     p.part_l, p.part_o,
                                     (std::size_t{seq} * attn::kKvHeads + kvh) * p.s_max + split,
                                     sh, false);
}

// The paged splits on one workgroup per CU (no reference counterpart): attn_ragged_stream_kernel
// over a paged cache, each tile's pages read from the page table one tile ahead of its copy.
// The partials equal attn_paged_split_kernel's (and the contiguous ragged ones) bit for bit; the
// same limits (attn_ragged_stream_fits).
template <int kBlock>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(1, 1)))
attn_paged_stream_kernel(AttnPagedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::StreamShared sh;
  decode_detail::PagedStreamSource src{p.k_pages, p.v_pages, p.page_table, p.max_pages,
                                       p.log2_page};
  decode_detail::stream_items(
      decode_detail::StreamBatch{p.q, p.part_m, p.part_l, p.part_o, p.lens, p.batch, p.s_max,
                                 attn_paged_len_cap(p.max_pages, p.log2_page), p.chunk},
      src, sh);
}

}  // namespace miso::kernels
