#pragma once

// Gated GQA softmax attention, prefill path, for MI355X (gfx950 / CDNA4): n consecutive tokens at
// positions pos0 .. pos0 + n - 1 of one sequence.
//   attn_prep_batch: the decode prep (norms, RoPE, KV append) for all n x 18 heads.
//   attn_prefill:    causal GQA flash attention with f16 MFMA (v_mfma_f32_32x32x16_f16), K/V
//                    tiles streamed into a 3-stage LDS ring by direct global->LDS loads, online
//                    softmax in f32 registers, sigmoid gate fused into the output store.
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
constexpr int kAttnQBlocksPerWave = 1;

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

constexpr int kKeys = 32;                      // keys per K/V tile (the M side of S^T = K Q^T)
constexpr int kStages = 3;                     // LDS ring depth: tiles i+1, i+2 load under tile i
constexpr int kRowBytes = attn::kDim * 2;      // 512: one f16 row
constexpr int kTileBytes = kKeys * kRowBytes;  // 16 KiB per K or V tile
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kRescaleSlack = 8.0f;  // log2 units: numerators stay <= 2^8 between rescales

struct Shared {
  alignas(16) unsigned char k[kStages][kTileBytes];
  alignas(16) unsigned char v[kStages][kTileBytes];
};

// 16-byte chunk c of tile row r lives at chunk position c ^ 2 (r % 16) of that row: 16 rows read
// at one chunk (S^T operands) and 4 rows read at two chunks (transpose reads) hit distinct banks.
__device__ inline unsigned swz(unsigned row, unsigned chunk) { return chunk ^ ((row & 15u) << 1); }

// This wave's share of the LDS loads of one tile: K and V rows 8 w .. 8 w + 7, one 1 KiB
// instruction per row pair and tensor (8 per wave). Rows past the last valid key are clamped
// into range and masked at use.
__device__ __attribute__((always_inline)) inline void load_tile(
    const attn::half_t* K, const attn::half_t* V, unsigned k0, unsigned last_row,
    unsigned k_lds, unsigned v_lds, unsigned wave, unsigned lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned m = wave * 4 + i;  // 1 KiB instruction index: rows 2m, 2m + 1
    const unsigned row = 2 * m + (lane >> 5);
    unsigned r = k0 + row;
    r = r < last_row ? r : last_row;
    const std::size_t at = std::size_t{r} * attn::kDim + swz(row, lane & 31u) * 8;
    cdna4::lds_load16(K + at, k_lds + m * 1024);
    cdna4::lds_load16(V + at, v_lds + m * 1024);
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
// owns tokens 16 b + 4 w .. + 4 as one MFMA column block of 32 query rows (row n = token offset
// n / 8, head n % 8).
//
// K/V tiles of 32 keys stream into a 3-stage LDS ring with direct global->LDS loads (no VGPR
// staging); one barrier per tile. Per tile each wave computes S^T = K Q^T (16 MFMAs over
// head_dim 256; Q^T resident in registers as f16,
// pre-scaled by 1/16), masks causally, updates the online softmax in log2 units on the lane's own
// query columns (rescaling the accumulators only when a max grows by more than 2^8), and
// accumulates O^T += V^T P^T (16 MFMAs: P^T stays in the S^T accumulator layout, V^T comes
// from ds_read_b64_tr_b16 with keys ordered to match). The gate and 1/l are applied at the store.
template <int kBlock>
__device__ void attn_prefill_op(const AttnPrefillParams& p, unsigned first, unsigned count) {
  using namespace prefill_detail;
  using attn::kDim;
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  constexpr int kGroup = attn::kQHeads / attn::kKvHeads;
  constexpr int kNB = kAttnQBlocksPerWave;  // 32-row MFMA column blocks per wave
  __shared__ Shared sh;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned col = lane & 31u, hi = lane >> 5;  // MFMA column / lane half
  const unsigned blocks = (p.n + kAttnQBlock - 1) / kAttnQBlock;
  const unsigned k_lds0 = cdna4::lds_offset(sh.k[0]), v_lds0 = cdna4::lds_offset(sh.v[0]);

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
    const unsigned tiles = (kv_end + kKeys - 1) / kKeys;

    // Start streaming before anything else: tiles 0 and 1.
    load_tile(K, V, 0, kv_end - 1, k_lds0, v_lds0, wave, lane);
    if (tiles > 1)
      load_tile(K, V, kKeys, kv_end - 1, k_lds0 + kTileBytes, v_lds0 + kTileBytes, wave, lane);

    // This lane's query rows: block nb -> token tq[nb], head kvh * 8 + hq.
    const unsigned tw = t0 + 4 * kNB * wave, hq = col % kGroup;
    unsigned tq[kNB], lim[kNB];
    bool q_valid[kNB];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const unsigned raw = tw + 4 * nb + col / kGroup;
      q_valid[nb] = raw < p.n;
      tq[nb] = q_valid[nb] ? raw : p.n - 1;
      lim[nb] = p.pos0 + tq[nb];  // last visible key
    }
    const bool wave_active = tw < p.n;
    const unsigned wave_lim = p.pos0 + min(tw + 4 * kNB - 1, p.n - 1);  // last key any row sees
    const unsigned wave_lim_lo = p.pos0 + tw;                 // every row sees keys <= this

    // Q^T operands: dims 16 s + 8 hi + j of the lane's rows, scaled by 1/16 (exact in f16).
    half8_t qb[kNB][16];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const float* src =
          p.q + (std::size_t{tq[nb]} * attn::kQHeads + kvh * kGroup + hq) * kDim + 8 * hi;
      const float z = q_valid[nb] ? 0.0625f : 0.0f;
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const float4 x0 = *reinterpret_cast<const float4*>(src + 16 * s);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 16 * s + 4);
        qb[nb][s] = half8_t{static_cast<_Float16>(x0.x * z), static_cast<_Float16>(x0.y * z),
                            static_cast<_Float16>(x0.z * z), static_cast<_Float16>(x0.w * z),
                            static_cast<_Float16>(x1.x * z), static_cast<_Float16>(x1.y * z),
                            static_cast<_Float16>(x1.z * z), static_cast<_Float16>(x1.w * z)};
      }
    }
    float16_t oacc[kNB][8];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
      for (int b = 0; b < 8; ++b)
        oacc[nb][b] = float16_t{};
    float m_run[kNB], l_run[kNB];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
      m_run[nb] = -__builtin_inff(), l_run[nb] = 0.0f;

    // Per-lane LDS byte offsets of the S^T (K) and P V (V^T, transpose) operands within a tile.
    const unsigned g = lane >> 4, j = lane & 15u;
    const unsigned vrow = 4 * (g >> 1) + j / 4;                   // + 16 step (+ 8 upper half)
    const unsigned vchunk = 2 * (g & 1u) + (j % 4) / 2;           // + 4 b
    const unsigned vbyte = 8 * ((j % 4) & 1u);

    for (unsigned ti = 0; ti < tiles; ++ti) {
      // Tile ti has landed once at most the 8 loads of tile ti + 1 are still in flight.
      if (ti + 1 < tiles)
        cdna4::wait_vmcnt<8>();
      else
        cdna4::wait_vmcnt<0>();
      __syncthreads();  // every wave's share of tile ti is in LDS; tile ti - 1 is fully read
      if (ti + 2 < tiles) {
        const unsigned st = (ti + 2) % kStages;
        load_tile(K, V, (ti + 2) * kKeys, kv_end - 1, k_lds0 + st * kTileBytes,
                  v_lds0 + st * kTileBytes, wave, lane);
      }
      const unsigned k0 = ti * kKeys, buf = ti % kStages;
      if (!wave_active || k0 > wave_lim)
        continue;  // wave-uniform: no row of this wave sees these keys
      const unsigned char* kt = sh.k[buf];
      const unsigned char* vt = sh.v[buf];

      // S^T[key][row] for 32 keys x 2 x 32 rows.
      float16_t sacc[kNB];
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb)
        sacc[nb] = float16_t{};
#pragma unroll
      for (int s = 0; s < 16; ++s) {
        const half8_t a =
            *reinterpret_cast<const half8_t*>(kt + col * kRowBytes + swz(col, 2 * s + hi) * 16);
#pragma unroll
        for (int nb = 0; nb < kNB; ++nb)
          sacc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[nb][s], sacc[nb], 0, 0, 0);
      }
      const bool full = k0 + kKeys - 1 <= wave_lim_lo;  // no key of the tile is masked
      half8_t pb[kNB][2];
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb) {
        float x[16];
        float mx = -__builtin_inff();
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
          x[r] = (full || key <= lim[nb]) ? sacc[nb][r] * kLog2e : -__builtin_inff();
          mx = fmaxf(mx, x[r]);
        }
        mx = cdna4::max_xor32(mx);
        // Lazy rescale: keep the reference max unless this tile exceeds it by the slack.
        if (__builtin_amdgcn_ballot_w64(mx > m_run[nb] + kRescaleSlack)) {
          const float m_new = fmaxf(m_run[nb], mx);
          const float corr = __builtin_amdgcn_exp2f(m_run[nb] - m_new);  // 0 on the first tile
          l_run[nb] *= corr;
#pragma unroll
          for (int b = 0; b < 8; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              oacc[nb][b][r] *= corr;
          m_run[nb] = m_new;
        }
        float ls = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pr = __builtin_amdgcn_exp2f(x[r] - m_run[nb]);
          ls += pr;
          pb[nb][r / 8][r % 8] = static_cast<_Float16>(pr);
        }
        l_run[nb] += ls;
      }
      // O^T[d][row] += V^T[d][key] P^T[key][row]; k-slot 8 hi + j <-> key 16 step + 4 hi +
      // (j < 4 ? j : j + 4), matching the S^T accumulator rows this lane holds.
#pragma unroll
      for (int step = 0; step < 2; ++step) {
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const unsigned r0 = 16 * step + vrow, r1 = r0 + 8, ch = 4 * b + vchunk;
          const half4_t lo = read_tr(vt + r0 * kRowBytes + swz(r0, ch) * 16 + vbyte);
          const half4_t up = read_tr(vt + r1 * kRowBytes + swz(r1, ch) * 16 + vbyte);
          const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
#pragma unroll
          for (int nb = 0; nb < kNB; ++nb)
            oacc[nb][b] =
                __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[nb][step], oacc[nb][b], 0, 0, 0);
        }
      }
    }
    __syncthreads();  // the ring is reused by the next item

    // Row totals: each column's keys per tile were split between the lane halves.
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const float l_tot = cdna4::sum_xor32(l_run[nb]);
      if (!q_valid[nb])
        continue;
      const unsigned head = kvh * kGroup + hq;
      const float inv_l = 1.0f / l_tot;
      const float* gate = p.qg + std::size_t{tq[nb]} * p.qg_stride + head * 2 * kDim + kDim;
      float* out = p.core + (std::size_t{tq[nb]} * attn::kQHeads + head) * kDim;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const unsigned d0 = 32 * b + 8 * r4 + 4 * hi;
          const float4 gv = *reinterpret_cast<const float4*>(gate + d0);
          float4 o;
          o.x = oacc[nb][b][4 * r4 + 0] * inv_l / (1.0f + __expf(-gv.x));
          o.y = oacc[nb][b][4 * r4 + 1] * inv_l / (1.0f + __expf(-gv.y));
          o.z = oacc[nb][b][4 * r4 + 2] * inv_l / (1.0f + __expf(-gv.z));
          o.w = oacc[nb][b][4 * r4 + 3] * inv_l / (1.0f + __expf(-gv.w));
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
