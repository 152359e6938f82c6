#pragma once

// Gated GQA softmax attention, prefill path, for MI355X (gfx950 / CDNA4): n consecutive tokens at
// positions pos0 .. pos0 + n - 1 of one sequence.
//   attn_prep_batch: the decode prep (norms, RoPE, KV append) for all n x 18 heads.
//   attn_prefill:    causal GQA flash attention with f16 MFMA (v_mfma_f32_32x32x16_f16), K/V
//                    tiles double-buffered in LDS, online softmax in f32 registers, sigmoid gate
//                    fused into the output store.
//
// Source-compatible drop-in for miso's kernels/attention_prefill.hpp (same structs, field order,
// kernel names and template parameters; attn_prefill_items sizes the caller's grid).

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "attention_decode.hpp"
#include "cdna4_wave.hpp"

namespace miso::kernels {

// ------------------------------------------------------------------------------------------------
// Batched prep (reference: kernels/attention_prefill.hpp:20-40)
// ------------------------------------------------------------------------------------------------

// Items [first, first + count) of 18 n (token-major).
template <int kBlock>
__device__ void attn_prep_batch_op(const AttnPrepBatchParams& p, unsigned first, unsigned count) {
  using namespace attn;
  constexpr unsigned kHeads = kQHeads + kKvHeads;
  for (unsigned item = first + blockIdx.x; item < first + count; item += gridDim.x) {
    const unsigned t = item / kHeads, head = item % kHeads;
    AttnPrepParams one = p.tok0;
    one.qg += std::size_t{t} * p.proj_stride;
    one.k += std::size_t{t} * p.proj_stride;
    one.v += std::size_t{t} * p.proj_stride;
    one.q += std::size_t{t} * kQHeads * kDim;
    one.pos += t;
    attn_prep_head<kBlock>(one, head);
  }
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prep_batch_kernel(AttnPrepBatchParams p) {
  attn_prep_batch_op<kBlock>(p, 0, p.n * (attn::kQHeads + attn::kKvHeads));
}

// ------------------------------------------------------------------------------------------------
// Causal prefill (reference: kernels/attention_prefill.hpp:42-161)
// ------------------------------------------------------------------------------------------------

struct AttnPrefillParams {
  const float* q;               // [n][16][256] normalised, rotated (unscaled)
  const float* qg;              // token-major; gate at tok * qg_stride + head * 512 + 256
  const attn::half_t* k_cache;  // [2][max_ctx][256], positions [0, pos0 + n) valid
  const attn::half_t* v_cache;
  float* core;  // [n][16][256]
  unsigned pos0, n, max_ctx;
  unsigned qg_stride;  // 8192 packed, or 9216 when q/k/v share a proj buffer
};

// Tokens per workgroup: 4 waves x 4 tokens x 8 query heads = 32 query rows per wave, the N side
// of one 32x32 MFMA tile.
constexpr unsigned kAttnQBlock = 16;

// Grid size. Items come in groups of 8 (one per XCD of the round-robin dispatch): slots 0-3 of a
// group serve KV head 0 and slots 4-7 KV head 1, so each XCD's L2 holds one KV head's stream, and
// ranks are handed out heaviest token block first. Slots past the last block exit at once.
__host__ __device__ inline unsigned attn_prefill_items(unsigned n) {
  const unsigned blocks = (n + kAttnQBlock - 1) / kAttnQBlock;
  return 8 * ((blocks + 3) / 4);
}

namespace prefill_detail {

using cdna4::float16_t;
using cdna4::half4_t;
using cdna4::half8_t;
typedef __fp16 lds_fp16x4 __attribute__((vector_size(8)));

constexpr int kKeys = 32;                   // keys per K/V tile (the M side of S^T = K Q^T)
constexpr int kKPitch = attn::kDim * 2 + 16;  // bytes per K row in LDS: 16-byte skew per row
constexpr int kVPitch = attn::kDim * 2 + 32;  // bytes per V row: 32-byte skew (transpose reads)
constexpr int kKTile = kKeys * kKPitch;
constexpr int kVTile = kKeys * kVPitch;
constexpr float kLog2e = 1.44269504088896340736f;

struct Shared {
  alignas(16) unsigned char k[2][kKTile];
  alignas(16) unsigned char v[2][kVTile];
};

// Global -> register staging of one K/V tile: 32 rows x 32 chunks of 16 bytes each for K and V;
// thread t moves chunks t + 256 i, i = 0..3 (row = chunk / 32), rows clamped into [0, kv_end).
struct Stage {
  uint4 k[4], v[4];
};

__device__ inline void stage_load(Stage& st, const attn::half_t* K, const attn::half_t* V,
                                  unsigned k0, unsigned last_row, unsigned t) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned id = t + 256u * i, row = id >> 5, col = id & 31u;
    unsigned r = k0 + row;
    r = r < last_row ? r : last_row;
    const std::size_t at = std::size_t{r} * attn::kDim + col * 8;
    st.k[i] = *reinterpret_cast<const uint4*>(K + at);
    st.v[i] = *reinterpret_cast<const uint4*>(V + at);
  }
}

__device__ inline void stage_store(const Stage& st, unsigned char* kl, unsigned char* vl,
                                   unsigned t) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned id = t + 256u * i, row = id >> 5, col = id & 31u;
    *reinterpret_cast<uint4*>(kl + row * kKPitch + col * 16) = st.k[i];
    *reinterpret_cast<uint4*>(vl + row * kVPitch + col * 16) = st.v[i];
  }
}

__device__ inline half4_t read_tr(const unsigned char* base) {
  const lds_fp16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      (__attribute__((address_space(3))) lds_fp16x4*)(base));
  return __builtin_bit_cast(half4_t, raw);
}

}  // namespace prefill_detail

// Items [first, first + count) (grid-stride). Item -> (KV head, token block) as described at
// attn_prefill_items. Per workgroup: tokens [16 b, 16 b + 16) x 8 heads of one KV head; wave w
// owns tokens 16 b + 4 w .. + 4 as 32 query rows (row n = token offset n / 8, head n % 8).
//
// Per 32-key tile each wave computes S^T = K Q^T (16 MFMAs over head_dim 256; K rows from LDS,
// Q^T resident in registers as f16, pre-scaled by 1/16), masks causally, updates the online
// softmax in log2 units on the lane's own query column, and accumulates O^T += V^T P^T (16 MFMAs:
// P^T stays in the S^T accumulator layout, V^T comes from LDS through ds_read_b64_tr_b16, keys
// ordered to match). The gate and 1/l are applied at the store.
template <int kBlock>
__device__ void attn_prefill_op(const AttnPrefillParams& p, unsigned first, unsigned count) {
  using namespace prefill_detail;
  using attn::kDim;
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  constexpr int kGroup = attn::kQHeads / attn::kKvHeads;
  __shared__ Shared sh;
  const unsigned t = threadIdx.x, lane = t & 63u, wave = t >> 6;
  const unsigned col = lane & 31u, hi = lane >> 5;  // MFMA column / lane half
  const unsigned blocks = (p.n + kAttnQBlock - 1) / kAttnQBlock;

  for (unsigned item = first + blockIdx.x; item < first + count; item += gridDim.x) {
    const unsigned slot = item % 8, kvh = slot / 4;
    const unsigned rank = (item / 8) * 4 + slot % 4;
    if (rank >= blocks)
      continue;  // uniform across the workgroup
    const unsigned blk = blocks - 1 - rank;
    const unsigned t0 = blk * kAttnQBlock;
    const unsigned t_end = min(t0 + kAttnQBlock, p.n);
    const unsigned kv_end = p.pos0 + t_end;
    const attn::half_t* K = p.k_cache + std::size_t{kvh} * p.max_ctx * kDim;
    const attn::half_t* V = p.v_cache + std::size_t{kvh} * p.max_ctx * kDim;

    // This lane's query row (MFMA column): token tq, head kvh * 8 + hq.
    const unsigned tw = t0 + 4 * wave;
    const unsigned tq_raw = tw + col / kGroup, hq = col % kGroup;
    const bool q_valid = tq_raw < p.n;
    const unsigned tq = q_valid ? tq_raw : p.n - 1;
    const unsigned lim = p.pos0 + tq;  // last visible key
    const unsigned wave_last_tok = min(tw + 3, p.n - 1);
    const bool wave_active = tw < p.n;
    const unsigned wave_lim = p.pos0 + wave_last_tok;

    // Q^T operand: dims 16 s + 8 hi + j of the lane's row, scaled by 1/16 (exact in f16).
    half8_t qb[16];
    {
      const float* src = p.q + (std::size_t{tq} * attn::kQHeads + kvh * kGroup + hq) * kDim + 8 * hi;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float4 x0 = *reinterpret_cast<const float4*>(src + 16 * s);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 16 * s + 4);
        const float z = q_valid ? 0.0625f : 0.0f;
        qb[s] = half8_t{static_cast<_Float16>(x0.x * z), static_cast<_Float16>(x0.y * z),
                        static_cast<_Float16>(x0.z * z), static_cast<_Float16>(x0.w * z),
                        static_cast<_Float16>(x1.x * z), static_cast<_Float16>(x1.y * z),
                        static_cast<_Float16>(x1.z * z), static_cast<_Float16>(x1.w * z)};
      }
    }
    float16_t oacc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b)
      oacc[b] = float16_t{};
    float m_run = -__builtin_inff(), l_run = 0.0f;

    const unsigned tiles = (kv_end + kKeys - 1) / kKeys;
    Stage stg;
    stage_load(stg, K, V, 0, kv_end - 1, t);
    stage_store(stg, sh.k[0], sh.v[0], t);
    __syncthreads();
    for (unsigned ti = 0; ti < tiles; ++ti) {
      const unsigned k0 = ti * kKeys, buf = ti & 1u;
      if (ti + 1 < tiles)
        stage_load(stg, K, V, k0 + kKeys, kv_end - 1, t);
      if (wave_active && k0 <= wave_lim) {
        // S^T[key][row] for 32 keys x 32 rows.
        float16_t sacc = float16_t{};
        const unsigned char* krow = sh.k[buf] + col * kKPitch + 16 * hi;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
          const half8_t a = *reinterpret_cast<const half8_t*>(krow + 32 * s);
          sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[s], sacc, 0, 0, 0);
        }
        // Causal mask and online softmax (log2 units) on this lane's 16 keys of the column.
        float x[16];
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
          x[r] = key <= lim ? sacc[r] * kLog2e : -__builtin_inff();
          mx = fmaxf(mx, x[r]);
        }
        mx = cdna4::max_xor32(mx);
        const float m_new = fmaxf(m_run, mx);  // finite: key 0 is visible to every row
        const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
        float ls = 0.0f;
        half8_t pb[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = __builtin_amdgcn_exp2f(x[r] - m_new);
          ls += pr;
          pb[r / 8][r % 8] = static_cast<_Float16>(pr);
        }
        l_run = l_run * corr + ls;
        m_run = m_new;
        if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
#pragma unroll
          for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              oacc[b][r] *= corr;
        }
        // O^T[d][row] += V^T[d][key] P^T[key][row]; k-slot 8 hi + j <-> key 16 step + 4 hi +
        // (j < 4 ? j : j + 4), matching the S^T accumulator rows held by this lane.
        const unsigned g = lane >> 4, j = lane & 15u;
        const unsigned char* vbase =
            sh.v[buf] + (4 * (g >> 1) + j / 4) * kVPitch + (16 * (g & 1u) + 4 * (j % 4)) * 2;
#pragma unroll
        for (int step = 0; step < 2; ++step) {
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const unsigned char* at = vbase + (16 * step) * kVPitch + 64 * b;
            const half4_t lo = read_tr(at), up = read_tr(at + 8 * kVPitch);
            const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
            oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[step], oacc[b], 0, 0, 0);
          }
        }
      }
      if (ti + 1 < tiles)
        stage_store(stg, sh.k[buf ^ 1u], sh.v[buf ^ 1u], t);
      __syncthreads();
    }

    // Row totals: the column's 32 keys per tile were split between lane halves.
    const float l_tot = cdna4::sum_xor32(l_run);
    if (q_valid) {
      const unsigned head = kvh * kGroup + hq;
      const float inv_l = 1.0f / l_tot;
      const float* gate = p.qg + std::size_t{tq} * p.qg_stride + head * 2 * kDim + kDim;
      float* out = p.core + (std::size_t{tq} * attn::kQHeads + head) * kDim;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const unsigned d0 = 32 * b + 8 * r4 + 4 * hi;
          const float4 gv = *reinterpret_cast<const float4*>(gate + d0);
          float4 o;
          o.x = oacc[b][4 * r4 + 0] * inv_l / (1.0f + __expf(-gv.x));
          o.y = oacc[b][4 * r4 + 1] * inv_l / (1.0f + __expf(-gv.y));
          o.z = oacc[b][4 * r4 + 2] * inv_l / (1.0f + __expf(-gv.z));
          o.w = oacc[b][4 * r4 + 3] * inv_l / (1.0f + __expf(-gv.w));
          *reinterpret_cast<float4*>(out + d0) = o;
        }
      }
    }
  }
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prefill_kernel(AttnPrefillParams p) {
  attn_prefill_op<kBlock>(p, 0, attn_prefill_items(p.n));
}

}  // namespace miso::kernels
