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

// One head of 18 (0..15 query heads, 16..17 KV heads) on a 256-thread workgroup, thread d owning
// dimension d. The sum of squares is a wave64 butterfly plus a 4-entry LDS exchange; the RoPE
// partner (d +- 32) is lane ^ 32 of wave 0, read through the lane crossbar, so no LDS staging.
template <int kBlock>
__device__ void attn_prep_head(const AttnPrepParams& p, unsigned head) {
  using namespace attn;
  static_assert(kBlock == kDim, "one thread per dimension");
  __shared__ float wave_ss[kBlock / cdna4::kLanes];
  const unsigned d = threadIdx.x;
  const bool is_q = head < static_cast<unsigned>(kQHeads);
  const unsigned kvh = head - kQHeads;
  float x = is_q ? p.qg[head * 2 * kDim + d] : p.k[kvh * kDim + d];
  const float ss_wave = cdna4::wave_allsum(x * x);
  if ((d & 63u) == 0)
    wave_ss[d >> 6] = ss_wave;
  __syncthreads();
  const float ss = (wave_ss[0] + wave_ss[1]) + (wave_ss[2] + wave_ss[3]);
  const float r = rsqrtf(ss / kDim + p.eps);
  x = x * r * (is_q ? p.q_norm[d] : p.k_norm[d]);
  if (d < static_cast<unsigned>(kRopeDim)) {  // wave 0 only: uniform for the crossbar read
    constexpr unsigned kHalf = kRopeDim / 2;
    const float partner = cdna4::lane_xor32(x);
    float s, c;
    sincosf(static_cast<float>(p.pos) * p.inv_freq[d % kHalf], &s, &c);
    x = d < kHalf ? x * c - partner * s : x * c + partner * s;
  }
  if (is_q) {
    p.q[head * kDim + d] = x;
  } else {
    const std::size_t at = (std::size_t{kvh} * p.max_ctx + p.pos) * kDim + d;
    p.k_cache[at] = static_cast<half_t>(x);
    p.v_cache[at] = static_cast<half_t>(p.v[kvh * kDim + d]);
  }
  __syncthreads();  // wave_ss is reused by the next head of a grid-stride loop
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

constexpr int kRing = 4;                    // units per wave in the LDS ring (4-wave workgroups)
constexpr unsigned kUnitBytes = 8192;       // 8 rows of K + 8 rows of V
constexpr float kRescaleSlack = 8.0f;       // log2 units: numerators stay <= 2^8 between rescales

// LDS of one split workgroup: each wave's ring of K/V units (direct global->LDS loads), the query
// rows, per-wave softmax numerators (f16 pairs); the cross-wave merge reuses the ring.
template <int W, int R>
struct SplitSharedT {
  static constexpr int kWaveCount = W, kRingUnits = R;
  union {
    unsigned char ring[W][R][kUnitBytes];
    struct {
      float o[W][kGroup][attn::kDim];
      float m[W][kGroup];
      float mt[W][kGroup];
      float l[W][kGroup];
    } merge;
  };
  float q[kGroup][attn::kDim];
  _Float16 p[W][2][2][kGroup][2];  // [wave][row parity][pair][head][row of the pair]
};
using SplitShared = SplitSharedT<kWaves, kRing>;  // 4 waves x 4 units: 136.5 KiB

// A unit: rows u0 + 2 i + (lane / 32), i = 0..3, bytes [16 c, 16 c + 16) of each row (c = lane %
// 32), for K and for V. In global memory each row pair is 1 KiB contiguous; in the ring slot,
// K row pair i is at byte 1024 i and V row pair i at 4096 + 1024 i, lane-linear, so a lane's 16
// bytes land exactly where it reads them back.
struct Unit {
  uint4 k[4], v[4];
};

__device__ __attribute__((always_inline)) inline void load_unit(
    const attn::half_t* K, const attn::half_t* V, unsigned u0, unsigned last_row,
    unsigned slot_lds, unsigned lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned row = u0 + 2 * i + (lane >> 5);
    row = row < last_row ? row : last_row;  // rows past the span are masked, never out of bounds
    const std::size_t at = std::size_t{row} * attn::kDim + (lane & 31u) * 8;
    cdna4::lds_load16(K + at, slot_lds + 1024 * i);
    cdna4::lds_load16(V + at, slot_lds + 4096 + 1024 * i);
  }
}

__device__ __attribute__((always_inline)) inline Unit read_unit(const unsigned char* slot,
                                                                unsigned lane) {
  Unit u;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u.k[i] = *reinterpret_cast<const uint4*>(slot + 1024 * i + 16 * lane);
    u.v[i] = *reinterpret_cast<const uint4*>(slot + 4096 + 1024 * i + 16 * lane);
  }
  return u;
}

// Wait until the unit whose loads were followed by `after` (< 4) more units' loads has landed.
__device__ __attribute__((always_inline)) inline void wait_units_after(unsigned after) {
  switch (after) {
    case 0: cdna4::wait_vmcnt<0>(); break;
    case 1: cdna4::wait_vmcnt<8>(); break;
    case 2: cdna4::wait_vmcnt<16>(); break;
    default: cdna4::wait_vmcnt<24>(); break;
  }
}

// Running state of one wave: head h's reference max m, true max mt (log2 units) and sum l live in
// the 8 lanes whose (lane % 32) / 4 == h; o[h][e] is this lane's share of head h at dims 8 c + e for
// its row parity. l and o are relative to m.
struct WaveState {
  float m, mt, l;
  float o[kGroup][8];
};

// Online-softmax update of one unit. qh[h][j]: the lane's query slice (dims 8c + 2j, 8c + 2j + 1)
// of head h, pre-scaled by log2(e)/16, as f16 pairs. The reference max m moves only when a score
// exceeds it by more than kRescaleSlack (then o and l are rescaled exactly), so numerators
// exp2(s - m) stay below 2^kRescaleSlack and most units skip the rescale.
__device__ __attribute__((always_inline)) inline void process_unit(
    WaveState& st, const Unit& u, const half2_t (&qh)[kGroup][4], unsigned u0, unsigned span_end,
    _Float16 (*pbuf)[2][kGroup][2], unsigned lane) {
  const unsigned c = lane & 31u, a = lane >> 5;
  // Scores: partial dot products over this lane's 8 dims, then a reduce-scatter over the 32
  // lanes of the row parity leaves the complete score of (head c / 4, row u0 + 2 (c % 4) + a).
  float part[32];
#pragma unroll
  for (int h = 0; h < kGroup; ++h) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 kw = u.k[i];
      float acc = __builtin_amdgcn_fdot2(qh[h][0], cdna4::as_half2(kw.x), 0.0f, false);
      acc = __builtin_amdgcn_fdot2(qh[h][1], cdna4::as_half2(kw.y), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[h][2], cdna4::as_half2(kw.z), acc, false);
      acc = __builtin_amdgcn_fdot2(qh[h][3], cdna4::as_half2(kw.w), acc, false);
      part[h * 4 + i] = acc;
    }
  }
  float s = cdna4::reduce_scatter32(part);
  const unsigned my_row = u0 + 2 * (c & 3u) + a;
  if (my_row >= span_end)
    s = -__builtin_inff();
  // Head max over its 8 lanes (quad of rows, both parities). Row u0 is always in the span, so
  // every head has at least one finite score.
  float mu = fmaxf(s, cdna4::dpp_mov<cdna4::kQuadXor1>(s));
  mu = fmaxf(mu, cdna4::dpp_mov<cdna4::kQuadXor2>(mu));
  mu = cdna4::max_xor32(mu);
  st.mt = fmaxf(st.mt, mu);
  if (__builtin_amdgcn_ballot_w64(mu > st.m + kRescaleSlack)) {  // wave-uniform branch
    const float m_new = fmaxf(st.m, mu);
    const float corr = __builtin_amdgcn_exp2f(st.m - m_new);  // 0 on the first unit (m = -inf)
    st.l *= corr;
    st.m = m_new;
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
      const float ch = cdna4::as_float(__builtin_amdgcn_readlane(cdna4::as_uint(corr), 4 * h));
#pragma unroll
      for (int e = 0; e < 8; ++e)
        st.o[h][e] *= ch;
    }
  }
  const float pj = __builtin_amdgcn_exp2f(s - st.m);  // 0 for masked rows
  st.l += pj;
  // Numerators to LDS as f16: slot [parity a][pair (row index % 2)][head][row index / 2].
  {
    const unsigned ri = c & 3u, h = c >> 2;
    pbuf[a][ri & 1u][h][ri >> 1] = static_cast<_Float16>(pj);
  }
  // P V: rows (i, i + 2) of the parity pair up in one dot2 per (head, dim).
  half2_t pp[2][kGroup];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int h = 0; h < kGroup; ++h)
      __builtin_memcpy(&pp[g][h], &pbuf[a][g][h][0], sizeof(half2_t));
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const unsigned r0[4] = {u.v[g].x, u.v[g].y, u.v[g].z, u.v[g].w};
    const unsigned r1[4] = {u.v[g + 2].x, u.v[g + 2].y, u.v[g + 2].z, u.v[g + 2].w};
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
        st.o[h][e] = __builtin_amdgcn_fdot2(pp[g][h], pv[e], st.o[h][e], false);
  }
}

// Partial (m, l, o) of keys [span.begin, span.end) for KV head kvh, written at `base` (=
// kvh * n_splits + split) in the reference's partial layout. Wave w streams units w, w + 4, ...
// of the span through its kRing-unit LDS ring (kRing - 1 units in flight while one is processed);
// the four waves merge through LDS at the end. Every vector-memory load of the kernel is a direct
// LDS load with an explicit wait.
template <class Shared>
__device__ __attribute__((always_inline)) inline void split_partial(
    const float* __restrict__ q, const attn::half_t* K, const attn::half_t* V, unsigned len,
    AttnSpan span, unsigned kvh, float* part_m, float* part_l, float* part_o, std::size_t base,
    Shared& sh) {
  constexpr int kW = Shared::kWaveCount, kR = Shared::kRingUnits;
  static_assert(kR >= 2 && kR <= 4 && kGroup % kW == 0, "ring depth / wave count");
  const unsigned t = threadIdx.x, lane = t & 63u, c = lane & 31u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned last_row = len - 1;
  constexpr unsigned kStride = kW * kAttnDecodeUnit;
  const unsigned first = span.begin + wave * kAttnDecodeUnit;
  const unsigned n_units = first < span.end ? (span.end - first + kStride - 1) / kStride : 0;
  const unsigned ring0 = cdna4::lds_offset(sh.ring[wave][0]);

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
      load_unit(K, V, first + k * kStride, last_row, ring0 + k * kUnitBytes, lane);
  wait_units_after(n_units < kR - 1 ? n_units : kR - 1);  // the query loads are older
  __syncthreads();

  half2_t qh[kGroup][4];
  constexpr float kScale = kLog2e / 16.0f;  // 1/sqrt(256) in log2 units
#pragma unroll
  for (int h = 0; h < kGroup; ++h) {
    const float4 x0 = *reinterpret_cast<const float4*>(&sh.q[h][8 * c]);
    const float4 x1 = *reinterpret_cast<const float4*>(&sh.q[h][8 * c + 4]);
    qh[h][0] = half2_t{static_cast<_Float16>(x0.x * kScale), static_cast<_Float16>(x0.y * kScale)};
    qh[h][1] = half2_t{static_cast<_Float16>(x0.z * kScale), static_cast<_Float16>(x0.w * kScale)};
    qh[h][2] = half2_t{static_cast<_Float16>(x1.x * kScale), static_cast<_Float16>(x1.y * kScale)};
    qh[h][3] = half2_t{static_cast<_Float16>(x1.z * kScale), static_cast<_Float16>(x1.w * kScale)};
  }
  WaveState st;
  st.m = -__builtin_inff();
  st.mt = -__builtin_inff();
  st.l = 0.0f;
#pragma unroll
  for (int h = 0; h < kGroup; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e)
      st.o[h][e] = 0.0f;

  for (unsigned k = 0; k < n_units; ++k) {
    const unsigned ahead = k + kR - 1;
    if (ahead < n_units)  // its slot held unit k - 1, already read back into registers
      load_unit(K, V, first + ahead * kStride, last_row, ring0 + (ahead % kR) * kUnitBytes,
                lane);
    const unsigned after = n_units - 1 - k;
    wait_units_after(after < kR - 1 ? after : kR - 1);
    const Unit u = read_unit(sh.ring[wave][k % kR], lane);
    process_unit(st, u, qh, first + k * kStride, span.end, sh.p[wave], lane);
  }

  // Wave totals: l over the head's 8 lanes; o over the two row parities. swap32 of heads
  // (h, h + 4) leaves head h's total in the low half and head h + 4's in the high half.
  float l = st.l + cdna4::dpp_mov<cdna4::kQuadXor1>(st.l);
  l += cdna4::dpp_mov<cdna4::kQuadXor2>(l);
  l = cdna4::sum_xor32(l);
  __syncthreads();  // every wave is done with its ring: the merge area aliases it
  {
    const unsigned a = lane >> 5;
#pragma unroll
    for (int h = 0; h < kGroup / 2; ++h) {
      float tot[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const cdna4::Pair pr = cdna4::swap32(st.o[h][e], st.o[h + kGroup / 2][e]);
        tot[e] = pr.a + pr.b;
      }
      float4* dst = reinterpret_cast<float4*>(&sh.merge.o[wave][h + a * (kGroup / 2)][8 * c]);
      dst[0] = float4{tot[0], tot[1], tot[2], tot[3]};
      dst[1] = float4{tot[4], tot[5], tot[6], tot[7]};
    }
  }
  if (lane < 32 && (c & 3u) == 0) {
    sh.merge.m[wave][c >> 2] = st.m;
    sh.merge.mt[wave][c >> 2] = st.mt;
    sh.merge.l[wave][c >> 2] = l;
  }
  __syncthreads();
  // Merge the waves relative to the split's true max M: the kW * 64 threads split into 8 heads x
  // kTh threads of kDims dims. The partial is then exactly (max, sum exp(s - max), sum exp(s -
  // max) v).
  {
    constexpr unsigned kTh = kW * 64 / kGroup, kDims = attn::kDim / kTh;
    const unsigned h = t / kTh, d0 = kDims * (t % kTh);
    float M = -__builtin_inff();
#pragma unroll
    for (int w = 0; w < kW; ++w)
      M = fmaxf(M, sh.merge.mt[w][h]);
    float L = 0.0f, o[kDims] = {};
    if (M != -__builtin_inff()) {
#pragma unroll
      for (int w = 0; w < kW; ++w) {
        const float sc = __builtin_amdgcn_exp2f(sh.merge.m[w][h] - M);
        L += sc * sh.merge.l[w][h];
#pragma unroll
        for (unsigned e = 0; e < kDims; ++e)
          o[e] += sc * sh.merge.o[w][h][d0 + e];
      }
    }
    const std::size_t at = base * kGroup + h;
    if (t % kTh == 0) {
      part_m[at] = M * kLn2;  // -inf stays -inf for an empty span
      part_l[at] = L;
    }
    float4* dst = reinterpret_cast<float4*>(part_o + at * attn::kDim + d0);
#pragma unroll
    for (unsigned e = 0; e < kDims; e += 4)
      dst[e / 4] = float4{o[e], o[e + 1], o[e + 2], o[e + 3]};
  }
  __syncthreads();  // LDS is reused by the next item
}

}  // namespace decode_detail

// Split-K flash decoding on wave64 VALU (no MFMA). Item = kvh * n_splits + split (grid-stride,
// as the reference). Each split's keys are streamed in 8-row units: every lane loads 16 bytes of
// K and of V per row-pair (1 KiB coalesced per wave instruction), scores use v_dot2_f32_f16
// against the lane's f16 query slice and a DPP/crossbar reduce-scatter, the online softmax runs
// in log2 units, and P V uses v_dot2_f32_f16 over row pairs. Output: the reference's partial
// layout, m in natural-log units.
template <int kBlock>
__device__ void attn_split_op(const AttnSplitParams& p, unsigned first, unsigned count) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::SplitShared sh;
  for (unsigned item = first + blockIdx.y * gridDim.x + blockIdx.x; item < first + count;
       item += gridDim.x * gridDim.y) {
    const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
    const attn::half_t* K = p.k_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
    const attn::half_t* V = p.v_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
    decode_detail::split_partial(p.q, K, V, p.len, attn_split_span(p.len, p.n_splits, split),
                                 kvh, p.part_m, p.part_l, p.part_o,
                                 std::size_t{kvh} * p.n_splits + split, sh);
  }
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_split_kernel(AttnSplitParams p) {
  attn_split_op<kBlock>(p, 0, attn::kKvHeads * p.n_splits);
}

// The same split partials from 512-thread workgroups (8 waves, two per SIMD, 2-unit rings): one
// workgroup per (KV head, split), grid dim3(n_splits, 2). A second resident wave per SIMD hides
// the dependency stalls of the first.
__global__ void __launch_bounds__(512) attn_split_wide_kernel(AttnSplitParams p) {
  __shared__ decode_detail::SplitSharedT<8, 2> sh;
  const unsigned item = blockIdx.y * gridDim.x + blockIdx.x;
  if (item >= attn::kKvHeads * p.n_splits)
    return;
  const unsigned kvh = item / p.n_splits, split = item % p.n_splits;
  const attn::half_t* K = p.k_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
  const attn::half_t* V = p.v_cache + std::size_t{kvh} * p.max_ctx * attn::kDim;
  decode_detail::split_partial(p.q, K, V, p.len, attn_split_span(p.len, p.n_splits, split), kvh,
                               p.part_m, p.part_l, p.part_o,
                               std::size_t{kvh} * p.n_splits + split, sh);
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

// The merge of one head at dimension d, computed by a full wave whose 64 lanes own 64 adjacent
// dimensions of the same head. The result follows the reference's frozen FP32 order exactly:
// M = max_c m_c; for c in split order w = __expf(m_c - M), L = fma(w, l_c, L), o = fma(w, o_c, o);
// core = o / L / (1 + __expf(-gate)). Split statistics are per head, hence the same for the whole
// wave: lane c of each 64-split chunk loads m_c, l_c and forms w_c (a max is order-free and w_c
// depends only on m_c and M), the wave publishes (w_c, l_c) through LDS, and every lane then runs
// the ordered FMA chain over the chunk with all 64 o_c loads already in flight. A chunk past the
// last split is padded with w = 0 and a clamped, finite o: fma(0, x, acc) == acc exactly, so the
// padding cannot change a bit. Every template variant and the batched path use this routine, so
// all are bit-identical to one another and to a one-thread-per-dimension serial loop.
struct CombineLds {
  float w[cdna4::kLanes], l[cdna4::kLanes];
};

__device__ __attribute__((always_inline)) inline float combine_wave(
    const float* __restrict__ pm, const float* __restrict__ pl, const float* __restrict__ po,
    unsigned n_splits, float gate, CombineLds& lds) {
  constexpr unsigned kChunk = cdna4::kLanes, kStride = kGroup;  // partial rows per split
  constexpr std::size_t kOStride = std::size_t{kStride} * attn::kDim;
  const unsigned lane = cdna4::lane_id();
  float M = -__builtin_inff();
  for (unsigned c = lane; c < n_splits; c += kChunk)
    M = fmaxf(M, pm[c * kStride]);
  M = cdna4::wave_allmax(M);
  const unsigned last = n_splits - 1;
  float L = 0.0f, o = 0.0f;
  for (unsigned base = 0; base < n_splits; base += kChunk) {
    float ov[kChunk];
#pragma unroll
    for (unsigned r = 0; r < kChunk; ++r) {
      const unsigned c = base + r < last ? base + r : last;
      ov[r] = po[c * kOStride];
    }
    const unsigned mine = base + lane;
    const float w_l = mine < n_splits ? __expf(pm[mine * kStride] - M) : 0.0f;
    const float l_l = mine < n_splits ? pl[mine * kStride] : 0.0f;
    lds.w[lane] = w_l;
    lds.l[lane] = l_l;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (unsigned r = 0; r < kChunk; r += 4) {
      const float4 w4 = *reinterpret_cast<const float4*>(&lds.w[r]);
      const float4 l4 = *reinterpret_cast<const float4*>(&lds.l[r]);
      L = __builtin_fmaf(w4.x, l4.x, L);
      o = __builtin_fmaf(w4.x, ov[r], o);
      L = __builtin_fmaf(w4.y, l4.y, L);
      o = __builtin_fmaf(w4.y, ov[r + 1], o);
      L = __builtin_fmaf(w4.z, l4.z, L);
      o = __builtin_fmaf(w4.z, ov[r + 2], o);
      L = __builtin_fmaf(w4.w, l4.w, L);
      o = __builtin_fmaf(w4.w, ov[r + 3], o);
    }
    __builtin_amdgcn_wave_barrier();  // the next chunk overwrites the broadcast slots
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
  for (unsigned item = first + blockIdx.x; item < first + count; item += gridDim.x) {
    const unsigned h = item / kTiles, d = (item % kTiles) * kBlock + threadIdx.x;
    const unsigned kvh = h / kGroup, hl = h % kGroup;
    const std::size_t i0 = std::size_t{kvh} * p.n_splits * kGroup + hl;
    p.core[h * kDim + d] = decode_detail::combine_wave(
        p.part_m + i0, p.part_l + i0, p.part_o + i0 * kDim + d, p.n_splits,
        p.qg[h * 2 * kDim + kDim + d], lds[threadIdx.x / cdna4::kLanes]);
  }
}

template <int kBlock, bool kPrepared = false, int kPipeline = 1>
__global__ void __launch_bounds__(kBlock) attn_combine_kernel(AttnCombineParams p) {
  attn_combine_op<kBlock, kPrepared, kPipeline>(p, 0, attn::kQHeads * (attn::kDim / kBlock));
}

// ------------------------------------------------------------------------------------------------
// Ragged batched decode (no reference counterpart: the reference is batch-1). Semantics per
// sequence = split + combine above, with a dense gate tensor.
// ------------------------------------------------------------------------------------------------

// Keys per split for the batched path: large enough that the partials stay a few percent of the
// KV bytes, small enough that a batch of long and short sequences balances across CUs.
constexpr unsigned kAttnRaggedChunk = 512;

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
};

// Splits of a sequence of len keys: one per kAttnRaggedChunk keys, at most s_max.
__host__ __device__ inline unsigned attn_ragged_seq_splits(unsigned len, unsigned s_max) {
  const unsigned n = (len + kAttnRaggedChunk - 1) / kAttnRaggedChunk;
  return n < s_max ? n : s_max;
}

// One workgroup per (sequence, KV head, split slot); slots past the sequence's split count exit.
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_ragged_split_kernel(AttnRaggedParams p) {
  static_assert(kBlock == 256, "four waves per split workgroup");
  __shared__ decode_detail::SplitShared sh;
  const unsigned item = blockIdx.x;
  const unsigned split = item % p.s_max, kvh = (item / p.s_max) % attn::kKvHeads;
  const unsigned seq = item / (p.s_max * attn::kKvHeads);
  if (seq >= p.batch)
    return;
  const unsigned len = p.lens[seq];
  const unsigned n_splits = attn_ragged_seq_splits(len, p.s_max);
  if (split >= n_splits)
    return;
  const std::size_t kv0 = p.kv_offsets[seq] + std::size_t{kvh} * len * attn::kDim;
  decode_detail::split_partial(p.q + std::size_t{seq} * attn::kQHeads * attn::kDim,
                               p.k_cache + kv0, p.v_cache + kv0, len,
                               attn_split_span(len, n_splits, split), kvh, p.part_m, p.part_l,
                               p.part_o, (std::size_t{seq} * attn::kKvHeads + kvh) * p.s_max + split,
                               sh);
}

// One 64-thread workgroup per (sequence, head, 64-dim tile); the merge is combine_wave's.
__global__ void __launch_bounds__(64) attn_ragged_combine_kernel(AttnRaggedParams p) {
  constexpr unsigned kGroup = attn::kQHeads / attn::kKvHeads, kTiles = attn::kDim / 64;
  const unsigned item = blockIdx.x;
  const unsigned seq = item / (attn::kQHeads * kTiles), h = (item / kTiles) % attn::kQHeads;
  const unsigned d = (item % kTiles) * 64 + threadIdx.x;
  if (seq >= p.batch)
    return;
  const std::size_t out = (std::size_t{seq} * attn::kQHeads + h) * attn::kDim + d;
  const unsigned n_splits = attn_ragged_seq_splits(p.lens[seq], p.s_max);
  if (n_splits == 0) {
    p.core[out] = 0.0f;
    return;
  }
  const unsigned kvh = h / kGroup, hl = h % kGroup;
  const std::size_t i0 = (std::size_t{seq} * attn::kKvHeads + kvh) * p.s_max * kGroup + hl;
  __shared__ decode_detail::CombineLds lds;
  p.core[out] = decode_detail::combine_wave(p.part_m + i0, p.part_l + i0,
                                           p.part_o + i0 * attn::kDim + d, n_splits, p.gate[out],
                                           lds);
}

}  // namespace miso::kernels
