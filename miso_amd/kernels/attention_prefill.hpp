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
#include <type_traits>

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

// Tokens per workgroup: 4 waves x 8 tokens x 8 query heads = 64 query rows per wave, two 32-row
// MFMA column blocks.
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
constexpr int kStages = 3;                     // LDS ring depth
constexpr int kRowBytes = attn::kDim * 2;      // 512: one f16 row
constexpr int kTileBytes = kKeys * kRowBytes;  // 16 KiB per K or V tile
constexpr int kNB = kAttnQBlocksPerWave;       // 32-row MFMA column blocks per wave
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kRescaleSlack = 8.0f;  // log2 units: numerators stay <= 2^8 between rescales

// K tiles in the first 48 KiB, V tiles in the next 48 KiB, so every operand address is a per-lane
// base plus a compile-time offset below 64 KiB (the ring slot is folded into the offset).
constexpr unsigned kVBase = kStages * kTileBytes;
// 1 KiB alignment keeps the base clear of the address bits the swizzle XORs (4-8).
struct alignas(1024) Shared {
  unsigned char kv[2 * kStages * kTileBytes];
};

// 16-byte chunk c of tile row r lives at chunk position c ^ 2 (r % 16) of that row: the 32 rows
// read at one chunk (S^T operands) and the transpose reads spread over the banks. The XOR only
// touches address bits 4-8, so operand addresses are lane bases XOR compile-time constants.
__device__ inline unsigned swz(unsigned row, unsigned chunk) { return chunk ^ ((row & 15u) << 1); }

// Global -> LDS copy of tile rows [8 w, 8 w + 8) of K and V (one 1 KiB instruction per row pair
// and tensor). `off[i]` is this lane's byte offset of instruction i inside a tile (row 8 w + 2 i +
// lane / 32, chunk swz(row, lane % 32)); kt / vt are the tile's first rows (wave-uniform), so the
// copy needs no per-tile address arithmetic. M0 is saved and restored.
__device__ __attribute__((always_inline)) inline void copy_tile(const void* kt, const void* vt,
                                                                const unsigned (&off)[4],
                                                                unsigned k_lds, unsigned v_lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %7\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %5\n\t"
      "s_add_u32 m0, %7, 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %5\n\t"
      "s_add_u32 m0, %7, 0x800\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %3, %5\n\t"
      "s_add_u32 m0, %7, 0xc00\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %4, %5\n\t"
      "s_mov_b32 m0, %8\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %6\n\t"
      "s_add_u32 m0, %8, 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %6\n\t"
      "s_add_u32 m0, %8, 0x800\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %3, %6\n\t"
      "s_add_u32 m0, %8, 0xc00\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %4, %6\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(off[0]), "v"(off[1]), "v"(off[2]), "v"(off[3]), "s"(kt), "s"(vt), "s"(k_lds),
        "s"(v_lds)
      : "memory", "scc");
}

// The same copy for the tile that crosses the end of the keys: rows past last_row are clamped to
// it (they are masked at use), so no load leaves [0, last_row]. Also 8 instructions.
__device__ __attribute__((always_inline)) inline void copy_tile_clamped(
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

__device__ __attribute__((always_inline)) inline half8_t lds_read_b128(unsigned addr) {
  return *reinterpret_cast<const __attribute__((address_space(3))) half8_t*>(addr);
}

__device__ __attribute__((always_inline)) inline half4_t read_tr(unsigned addr) {
  const lds_fp16x4 raw = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
      reinterpret_cast<__attribute__((address_space(3))) lds_fp16x4*>(addr));
  return __builtin_bit_cast(half4_t, raw);
}

// Per-lane state of one wave: 64 query rows as two 32-row column blocks.
struct Rows {
  half8_t q[kNB][16];  // Q^T B operands: dims 16 s + 8 hi + j of the lane's rows, x log2(e)/16
  float m[kNB], l[kNB];
};

// S^T[key][row] = K Q^T for one tile (32 keys x 64 rows): 16 k-steps over head_dim, each K
// operand read once and used by both column blocks. kb: the lane's operand address in the tile's
// slot before the per-step XOR.
__device__ __attribute__((always_inline)) inline void scores(float16_t (&s)[kNB], const Rows& rw,
                                                            unsigned kb) {
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb)
    s[nb] = float16_t{};
#pragma unroll
  for (unsigned st = 0; st < 16; ++st) {
    const half8_t a = lds_read_b128(kb ^ (32u * st));
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
      s[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, rw.q[nb][st], s[nb], 0, 0, 0);
  }
}

// O^T[d][row] += V^T[d][key] P^T[key][row] for one tile; k-slot 8 hi + j of a step holds key
// 16 step + 4 hi + (j < 4 ? j : j + 4), which is how the S^T accumulator rows lie in the lane, so
// P^T is the softmax output as is. vb[b][u]: the lane's transpose-read addresses for 32-dim block
// b (u = 1: rows + 8) in tile slot 0; slot_off moves them to the tile's slot.
__device__ __attribute__((always_inline)) inline void accumulate(float16_t (&o)[kNB][8],
                                                                const half8_t (&p)[kNB][2],
                                                                const unsigned (&vb)[8][2],
                                                                unsigned slot_off) {
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const unsigned a0 = vb[b][0] + slot_off, a1 = vb[b][1] + slot_off;
#pragma unroll
    for (unsigned step = 0; step < 2; ++step) {
      const half4_t lo = read_tr(a0 + 8192u * step);
      const half4_t up = read_tr(a1 + 8192u * step);
      const half8_t a = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
#pragma unroll
      for (int nb = 0; nb < kNB; ++nb)
        o[nb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, p[nb][step], o[nb][b], 0, 0, 0);
    }
  }
}

// Online softmax of one tile's scores (log2 units) into f16 numerators. kMasked: key k0 + key(r)
// is visible to the lane's row nb iff it is <= lim[nb]. The reference max moves only when a tile
// exceeds it by more than the slack; that wave-uniform case returns true after setting `corr`
// (the factor the accumulators must be scaled by before the next tile is added).
template <bool kMasked>
__device__ __attribute__((always_inline)) inline bool softmax(const float16_t (&s)[kNB],
                                                             Rows& rw, half8_t (&p)[kNB][2],
                                                             float (&corr)[kNB], unsigned k0,
                                                             const unsigned (&lim)[kNB],
                                                             unsigned hi) {
  float x[kNB][16], mx[kNB];
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      x[nb][r] = s[nb][r];
  }
  if (kMasked) {  // the diagonal tiles only
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
        x[nb][r] = key <= lim[nb] ? x[nb][r] : -__builtin_inff();
      }
  }
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb) {
    float a = fmaxf(fmaxf(x[nb][0], x[nb][1]), x[nb][2]);
#pragma unroll
    for (int r = 3; r < 15; r += 2)
      a = fmaxf(fmaxf(a, x[nb][r]), x[nb][r + 1]);
    mx[nb] = fmaxf(a, x[nb][15]);
  }
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb)
    mx[nb] = cdna4::max_xor32(mx[nb]);  // the other 16 keys of the column are in lane ^ 32
  bool need = false;
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb)
    need |= mx[nb] > rw.m[nb] + kRescaleSlack;
  const bool rescale = __builtin_amdgcn_ballot_w64(need) != 0;
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb) {
    const float m_new = rescale ? fmaxf(rw.m[nb], mx[nb]) : rw.m[nb];
    corr[nb] = __builtin_amdgcn_exp2f(rw.m[nb] - m_new);  // 0 on the first tile (m = -inf)
    rw.m[nb] = m_new;
    float ls = 0.0f;
    float e[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      e[r] = __builtin_amdgcn_exp2f(x[nb][r] - m_new);  // 0 for masked keys
      ls += e[r];
    }
    rw.l[nb] = rw.l[nb] * corr[nb] + ls;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      p[nb][h] = half8_t{static_cast<_Float16>(e[8 * h + 0]), static_cast<_Float16>(e[8 * h + 1]),
                         static_cast<_Float16>(e[8 * h + 2]), static_cast<_Float16>(e[8 * h + 3]),
                         static_cast<_Float16>(e[8 * h + 4]), static_cast<_Float16>(e[8 * h + 5]),
                         static_cast<_Float16>(e[8 * h + 6]), static_cast<_Float16>(e[8 * h + 7])};
  }
  return rescale;
}

// o *= c for accumulators that live in AGPRs, element by element in place (read to a VGPR,
// multiply, write back). Written as assembly so the AGPR -> VGPR copies stay inside the caller's
// (rarely taken) branch: plain C++ lets the compiler hoist all 128 copies to the loop head.
__device__ __attribute__((always_inline)) inline void scale_acc(float16_t (&o)[8], float c) {
#pragma unroll
  for (int b = 0; b < 8; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float x = o[b][r], tmp;
      asm volatile(
          "v_accvgpr_read_b32 %1, %0\n\t"
          "v_mul_f32 %1, %1, %2\n\t"
          "v_accvgpr_write_b32 %0, %1"
          : "+a"(x), "=&v"(tmp)
          : "v"(c));
      o[b][r] = x;
    }
}

// One fully visible tile, software-pipelined (one column block per wave): the online softmax
// of tile ti (scores s, complete) gives P(ti); the scores of tile ti + 1 accumulate into s_next
// from the K operands at kb (ring slot of tile ti + 1); O += V^T(ti) P(ti) reads V at vb + v_off.
// The MFMAs are interleaved with the softmax VALU work and the LDS reads run two operands ahead,
// in a fixed order (scheduling barriers between the groups):
//   group 1: row max, rescale decision, S steps 0-1;  [rescale of O, rarely]
//   group 2: S steps 2-9, each with two exponentials and the running sums;
//   group 3: the 16 P V MFMAs with S steps 10-15 between them.
// m, l and O are updated in place (O rescaled before P(ti) is added). kMasked: keys k0 + key(r)
// past the row's causal limit lim (the diagonal tiles) are excluded; kNext: tile ti + 1 exists
// for this wave (otherwise no S MFMAs are issued).
template <bool kMasked, bool kNext>
__device__ __attribute__((always_inline)) inline void tile_step(float16_t& s, float16_t& s_next,
                                                               Rows& rw, float16_t (&o)[8],
                                                               unsigned kb,
                                                               const unsigned (&vb)[8][2],
                                                               unsigned v_off, unsigned k0,
                                                               unsigned lim, unsigned hi) {
  static_assert(kNB == 1, "the pipelined tile handles one column block");
  const half8_t(&q)[16] = rw.q[0];
  half8_t ka[16];
  auto kread = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext)
      ka[st] = lds_read_b128(kb ^ (32u * st));
  };
  auto smma = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext)
      s_next = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[st], q[st],
                                                      st == 0 ? float16_t{} : s_next, 0, 0, 0);
  };
  // Group 1.
  kread(0);
  kread(1);
  if (kMasked) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
      s[r] = key <= lim ? s[r] : -__builtin_inff();
    }
  }
  float a = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2)
    a = fmaxf(fmaxf(a, s[r]), s[r + 1]);
  const float mx = cdna4::max_xor32(fmaxf(a, s[15]));
  const bool rescale = __builtin_amdgcn_ballot_w64(mx > rw.m[0] + kRescaleSlack) != 0;
  const float m_new = rescale ? fmaxf(rw.m[0], mx) : rw.m[0];
  const float corr = __builtin_amdgcn_exp2f(rw.m[0] - m_new);
  rw.m[0] = m_new;
  kread(2);
  smma(0);
  kread(3);
  smma(1);
  __builtin_amdgcn_sched_barrier(0);
  if (rescale)
    scale_acc(o, corr);
  // Group 2: numerators of tile ti under S steps 2-9.
  float e[16], ls = 0.0f;
#pragma unroll
  for (unsigned st = 2; st < 10; ++st) {
    kread(st + 2);
    smma(st);
    const unsigned r = 2 * (st - 2);
    e[r] = __builtin_amdgcn_exp2f(s[r] - m_new);
    e[r + 1] = __builtin_amdgcn_exp2f(s[r + 1] - m_new);
    ls += e[r] + e[r + 1];
    __builtin_amdgcn_sched_barrier(0);
  }
  rw.l[0] = rw.l[0] * corr + ls;
  half8_t p[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    p[h] = half8_t{static_cast<_Float16>(e[8 * h + 0]), static_cast<_Float16>(e[8 * h + 1]),
                   static_cast<_Float16>(e[8 * h + 2]), static_cast<_Float16>(e[8 * h + 3]),
                   static_cast<_Float16>(e[8 * h + 4]), static_cast<_Float16>(e[8 * h + 5]),
                   static_cast<_Float16>(e[8 * h + 6]), static_cast<_Float16>(e[8 * h + 7])};
  // Group 3: P V, 32-dim block b and key step; V^T operands read four MFMAs ahead.
  constexpr unsigned kAhead = 4;
  half4_t vlo[kAhead], vup[kAhead];
  auto vread = [&](unsigned i) __attribute__((always_inline)) {
    const unsigned b = i / 2, step = i % 2;
    vlo[i % kAhead] = read_tr(vb[b][0] + v_off + 8192u * step);
    vup[i % kAhead] = read_tr(vb[b][1] + v_off + 8192u * step);
  };
#pragma unroll
  for (unsigned i = 0; i < kAhead; ++i)
    vread(i);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (unsigned i = 0; i < 16; ++i) {
    const half4_t lo = vlo[i % kAhead], up = vup[i % kAhead];
    const half8_t av = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
    if (i + kAhead < 16)
      vread(i + kAhead);
    o[i / 2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, p[i % 2], o[i / 2], 0, 0, 0);
    if (i % 3 == 0 && 10 + i / 3 < 16) {  // S steps 10-15 after P V MFMAs 0, 3, ..., 15
      const unsigned st = 10 + i / 3;
      if (st + 2 < 16)
        kread(st + 2);
      smma(st);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

__device__ __attribute__((always_inline)) inline void rescale_o(float16_t (&o)[kNB][8],
                                                               const float (&corr)[kNB]) {
#pragma unroll
  for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
    for (int b = 0; b < 8; ++b)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        o[nb][b][r] *= corr[nb];
}

}  // namespace prefill_detail

// Items [first, first + count) (grid-stride). Item -> (KV head, token block) as described at
// attn_prefill_items. Per workgroup: tokens [32 b, 32 b + 32) x 8 heads of one KV head; wave w
// owns tokens 32 b + 8 w .. + 8 as two MFMA column blocks of 32 query rows (row n = token offset
// n / 8, head n % 8).
//
// K/V tiles of 32 keys stream into a 3-stage LDS ring by direct global->LDS loads; one barrier
// per tile. Software pipeline per tile i: S^T(i + 1) = K Q^T (32 MFMAs, each K operand feeding
// both column blocks, Q^T resident as f16 pre-scaled by log2(e)/16), then O^T += V^T P^T(i) (32
// MFMAs, V^T from ds_read_b64_tr_b16), then the online softmax of tile i + 1 -- independent of
// the P V MFMAs, so it runs under them. Keys past a row's causal limit are masked only in the
// (at most two) diagonal tiles of a wave; the gate and 1/l are applied at the store.
template <int kBlock>
__device__ void attn_prefill_op(const AttnPrefillParams& p, unsigned first, unsigned count) {
  using namespace prefill_detail;
  using attn::kDim;
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  constexpr int kGroup = attn::kQHeads / attn::kKvHeads;
  constexpr unsigned kWaveTokens = 4 * kNB;
  __shared__ Shared sh;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned col = lane & 31u, hi = lane >> 5;  // MFMA column / lane half
  const unsigned blocks = (p.n + kAttnQBlock - 1) / kAttnQBlock;
  const unsigned lds0 = cdna4::lds_offset(sh.kv);

  // Per-lane constant addresses. Copy: instruction i moves rows 8 w + 2 i + lane / 32.
  unsigned copy_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned row = 8 * wave + 2 * i + (lane >> 5);
    copy_off[i] = row * kRowBytes + swz(row, lane & 31u) * 16;
  }
  // S^T A operand (key row col, chunk 2 st + hi): (col 512 + 16 hi + 32 (col % 16)) ^ 32 st.
  const unsigned kb = lds0 + col * kRowBytes + 16 * hi + 32 * (col & 15u);
  // V^T transpose reads: rows 16 step + vrow (+ 8), chunk 4 b + vchunk, byte vbyte, i.e.
  // (512 vrow + vbyte + 16 (vchunk ^ 2 vrow)) ^ (64 b) [^ 256, + 4096 for rows + 8] + 8192 step.
  unsigned vb[8][2];  // tile slot 0; + slot * 16 KiB for the others
  {
    const unsigned g = lane >> 4, j = lane & 15u;
    const unsigned vrow = 4 * (g >> 1) + j / 4, vchunk = 2 * (g & 1u) + (j % 4) / 2;
    const unsigned vbyte = 8 * ((j % 4) & 1u);
    const unsigned base = vrow * kRowBytes + vbyte + 16 * (vchunk ^ (2 * vrow));
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      vb[b][0] = lds0 + kVBase + (base ^ (64u * b));
      vb[b][1] = lds0 + kVBase + 4096 + (base ^ (64u * b) ^ 256u);
    }
  }

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
    auto copy = [&](unsigned ti) __attribute__((always_inline)) {
      const unsigned st = ti % kStages;
      const unsigned k_lds = lds0 + st * kTileBytes + wave * 4096;
      const unsigned v_lds = lds0 + kVBase + st * kTileBytes + wave * 4096;
      if ((ti + 1) * kKeys <= kv_end)
        copy_tile(K + std::size_t{ti} * kKeys * kDim, V + std::size_t{ti} * kKeys * kDim,
                  copy_off, k_lds, v_lds);
      else
        copy_tile_clamped(K, V, ti * kKeys, kv_end - 1, k_lds - wave * 4096,
                          v_lds - wave * 4096, wave, lane);
    };

    // Start streaming before anything else: tiles 0 and 1.
    copy(0);
    if (tiles > 1)
      copy(1);

    // This wave's rows: block nb -> token tq[nb] = tw + 4 nb + col / 8, head kvh * 8 + col % 8.
    const unsigned tw = t0 + kWaveTokens * wave, hq = col % kGroup;
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
    // Tiles this wave needs, and how many of them every row of the wave sees in full.
    const unsigned wave_tiles =
        wave_active ? (p.pos0 + min(tw + kWaveTokens - 1, p.n - 1)) / kKeys + 1 : 0;
    const unsigned full_tiles = wave_active ? (p.pos0 + tw + 1) / kKeys : 0;

    Rows rw;
    constexpr float kScale = kLog2e / 16.0f;  // 1/sqrt(256) in log2 units
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const float* src =
          p.q + (std::size_t{tq[nb]} * attn::kQHeads + kvh * kGroup + hq) * kDim + 8 * hi;
      const float z = q_valid[nb] ? kScale : 0.0f;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float4 x0 = *reinterpret_cast<const float4*>(src + 16 * st);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 16 * st + 4);
        rw.q[nb][st] = half8_t{static_cast<_Float16>(x0.x * z), static_cast<_Float16>(x0.y * z),
                               static_cast<_Float16>(x0.z * z), static_cast<_Float16>(x0.w * z),
                               static_cast<_Float16>(x1.x * z), static_cast<_Float16>(x1.y * z),
                               static_cast<_Float16>(x1.z * z), static_cast<_Float16>(x1.w * z)};
      }
      rw.m[nb] = -__builtin_inff();
      rw.l[nb] = 0.0f;
    }
    float16_t oacc[kNB][8];
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb)
#pragma unroll
      for (int b = 0; b < 8; ++b)
        oacc[nb][b] = float16_t{};
    half8_t pb[kNB][2];
    float corr[kNB];

    // Start of iteration ti: tile ti + 1 complete in LDS -- this wave's share by vmcnt (it is the
    // only copy in flight), every wave's by the barrier, which also says that all waves are done
    // with tile ti - 1, whose slot then receives tile ti + 2.
    auto sync_copy = [&](unsigned ti) __attribute__((always_inline)) {
      if (ti + 1 < tiles) {
        cdna4::wait_vmcnt<0>();
        __syncthreads();
        if (ti + 2 < tiles)
          copy(ti + 2);
      }
    };

    cdna4::wait_vmcnt<0>();  // tiles 0 (and 1) and the queries are in
    __syncthreads();
    // s: the scores of tile ti at the top of iteration ti (tile 0: computed here).
    float16_t s[kNB];
    if (wave_tiles > 0)
      scores(s, rw, kb);
    // One pass over the workgroup's tiles in three phases per wave, each a loop with a single
    // body (the per-wave bounds differ; every wave still runs sync_copy once per tile, in order):
    // the tiles its rows see in full, then its diagonal tiles (the last one has no successor),
    // then the tiles it does not need.
    float16_t s_next;
    unsigned ti = 0;
    for (; ti < full_tiles; ++ti) {
      sync_copy(ti);
      tile_step<false, true>(s[0], s_next, rw, oacc[0], kb + ((ti + 1) % kStages) * kTileBytes, vb,
                             (ti % kStages) * kTileBytes, 0, 0, hi);
      s[0] = s_next;
    }
    for (; ti + 1 < wave_tiles; ++ti) {
      sync_copy(ti);
      tile_step<true, true>(s[0], s_next, rw, oacc[0], kb + ((ti + 1) % kStages) * kTileBytes, vb,
                            (ti % kStages) * kTileBytes, ti * kKeys, lim[0], hi);
      s[0] = s_next;
    }
    if (ti < wave_tiles) {
      sync_copy(ti);
      tile_step<true, false>(s[0], s_next, rw, oacc[0], 0, vb, (ti % kStages) * kTileBytes,
                             ti * kKeys, lim[0], hi);
      ++ti;
    }
    for (; ti < tiles; ++ti)
      sync_copy(ti);
    __syncthreads();  // the ring is reused by the next item

    // Row totals: each column's keys per tile were split between the lane halves.
#pragma unroll
    for (int nb = 0; nb < kNB; ++nb) {
      const float l_tot = cdna4::sum_xor32(rw.l[nb]);
      if (!q_valid[nb])
        continue;
      const unsigned head = kvh * kGroup + hq;
      const float inv_l = __builtin_amdgcn_rcpf(l_tot);
      const float* gate = p.qg + std::size_t{tq[nb]} * p.qg_stride + head * 2 * kDim + kDim;
      float* out = p.core + (std::size_t{tq[nb]} * attn::kQHeads + head) * kDim;
#pragma unroll
      for (int b = 0; b < 8; ++b) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const unsigned d0 = 32 * b + 8 * r4 + 4 * hi;
          const float4 gv = *reinterpret_cast<const float4*>(gate + d0);
          float4 o;
          o.x = oacc[nb][b][4 * r4 + 0] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-gv.x));
          o.y = oacc[nb][b][4 * r4 + 1] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-gv.y));
          o.z = oacc[nb][b][4 * r4 + 2] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-gv.z));
          o.w = oacc[nb][b][4 * r4 + 3] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-gv.w));
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
