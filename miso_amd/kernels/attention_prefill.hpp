#pragma once

// Gated GQA softmax attention, prefill path, for MI355X (gfx950 / CDNA4): n consecutive tokens at
// positions pos0 .. pos0 + n - 1 of one sequence.
//   attn_prep_batch: the decode prep (norms, RoPE, KV append) for all n x 18 heads.
//   attn_prefill:    causal GQA flash attention with f16 MFMA (v_mfma_f32_32x32x16_f16), K/V
//                    tiles streamed into a 3-stage LDS ring by direct global->LDS loads, online
//                    softmax in f32 registers, sigmoid gate fused into the output store.
//
// Source-compatible drop-in for miso's kernels/attention_prefill.hpp (same structs, field order,
// kernel names and template parameters; attn_prefill_items sizes the caller's grid). The MFMAs
// are issued from inline assembly so that O holds the AGPR file and the scores stay in VGPRs;
// the wait states the compiler would add around them are explicit (drain_pv, the step's s_nop).

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

// Tokens per workgroup. Each wave owns 4 tokens x 8 query heads per 32-row MFMA column block;
// short launches give each wave one block (16 tokens per workgroup, so more workgroups share a
// causal prefill), launches of kAttnWideMin tokens or more two blocks (32 tokens per workgroup:
// each K and V operand read from LDS feeds two MFMAs).
constexpr unsigned kAttnQBlock = 16;
constexpr unsigned kAttnWideMin = 4096;
__host__ __device__ constexpr unsigned attn_prefill_row_blocks(unsigned n) {
  return n >= kAttnWideMin ? 2 : 1;
}

// Grid size. Items come in groups of 8 (one per XCD of the round-robin dispatch): slots 0-3 of a
// group serve KV head 0 and slots 4-7 KV head 1, so each XCD's L2 holds one KV head's stream, and
// ranks are handed out heaviest token block first. Slots past the last block exit at once.
__host__ __device__ inline unsigned attn_prefill_items(unsigned n) {
  const unsigned tokens = kAttnQBlock * attn_prefill_row_blocks(n);
  const unsigned blocks = (n + tokens - 1) / tokens;
  return 8 * ((blocks + 3) / 4);
}

// ------------------------------------------------------------------------------------------------
// Balanced causal prefill (no reference counterpart; the reference launches one workgroup per
// token block). Under a causal mask block b of a launch sees ~b tiles of keys, so with one
// workgroup per block the last block sets the time at about twice the mean. For launches of up
// to 4096 tokens the balanced form pairs block B-1-j with block j (their tile counts sum to a
// near constant) and gives the pair two workgroups: A takes the heavy block's first
// S = ceil(pair tiles / 2) tiles, B the heavy block's remaining tiles and then the light block.
// Both parts of a split block write their partial (m, l, O) to a workspace; whichever finishes
// second (an agent-scope counter per pair) merges the other's partial into its own and stores
// the output.
// Pairs whose heavy block would save fewer than kAttnSplitMinTiles tiles run unsplit (A: the
// heavy block, B: the light one). The pairing pays while its grid fits the chip at one
// workgroup per CU (256 on an MI355X): one row block per wave (16-token blocks) up to 2048
// tokens, two (32-token blocks) from 3841 to 4096 (attn_prefill_balanced). Otherwise the
// one-workgroup-per-block layout's extra rounds already even out the load (measured: 3072 tokens
// after a 1024-token prefix in 16-token pairs, 384 workgroups, 202 us against 175 us).
// ------------------------------------------------------------------------------------------------

constexpr unsigned kAttnSplitMinTiles = 4;
// Tiles moved from B's share of a split pair to A's, for 16- and 32-token blocks (B pays a second
// query prologue and the light block's output; measured best: none with 16-token blocks, ~1%
// for 4 with 32-token blocks).
constexpr unsigned kAttnSplitBias = 0, kAttnSplitBias2 = 4;
constexpr unsigned kAttnBalancedMaxItems = 256;  // CUs of an MI355X

// Workspace of the balanced form: one counter per pair (a fixed region of kAttnSplitMaxPairs, so
// one workspace serves every n), then (m, l) (f32 [slot][rows][2]) and O (f32 [slot][rows][256])
// of the two parts (slots 2 pair, 2 pair + 1) of each pair, rows = 128 per row block per wave.
// The counters must be zero before the first launch over a workspace; every launch leaves them
// zero. Launches that overlap on one workspace race.
struct AttnPrefillSplitParams {
  AttnPrefillParams a;
  float* part_o;
  float* part_ml;
  unsigned* counters;
};

// Row blocks per wave of the balanced form: one up to 2048 tokens, two up to 4096.
__host__ __device__ constexpr unsigned attn_prefill_balanced_blocks(unsigned n) {
  return n > 2048 ? 2 : 1;
}
__host__ __device__ constexpr unsigned attn_prefill_split_block_count(unsigned n) {
  const unsigned tokens = kAttnQBlock * attn_prefill_balanced_blocks(n);
  return (n + tokens - 1) / tokens;
}
__host__ __device__ constexpr unsigned attn_prefill_split_pairs(unsigned n) {
  return attn::kKvHeads * (attn_prefill_split_block_count(n) / 2);
}
// Rows of one part's partial: 128 query rows per row block.
__host__ __device__ constexpr unsigned attn_prefill_split_rows(unsigned n) {
  return 128 * attn_prefill_balanced_blocks(n);
}
constexpr unsigned kAttnSplitMaxPairs = attn::kKvHeads * (kAttnWideMin / kAttnQBlock / 2);
constexpr std::size_t kAttnSplitCounterBytes = kAttnSplitMaxPairs * sizeof(unsigned);

// Grid size: per KV head one slot per pair (and one for the middle block of an odd count),
// groups of 4 slots per XCD pair round (XCD = item % 8 as in attn_prefill_items), the two
// workgroups of a slot in consecutive rounds on the same XCD.
__host__ __device__ constexpr unsigned attn_prefill_split_items(unsigned n) {
  const unsigned blocks = attn_prefill_split_block_count(n);
  const unsigned slots = blocks / 2 + blocks % 2;
  return 16 * ((slots + 3) / 4);
}

// Whether a launch of n tokens takes the balanced form: n <= 2048 (16-token blocks) or, with
// 32-token blocks, when the grid fills the chip (3841 <= n <= 4096); between the two the
// one-block-per-workgroup layout over two rounds is faster (3072 tokens on an empty cache:
// 121.6 us against 151.9 us for 192 paired workgroups).
__host__ __device__ constexpr bool attn_prefill_balanced(unsigned n) {
  return n > 0 && n <= kAttnWideMin && attn_prefill_split_items(n) <= kAttnBalancedMaxItems &&
         (n <= 2048 || attn_prefill_split_items(n) == kAttnBalancedMaxItems);
}

__host__ __device__ constexpr std::size_t attn_prefill_split_workspace_bytes(unsigned n) {
  return kAttnSplitCounterBytes + std::size_t{attn_prefill_split_pairs(n)} * 2 *
                                      attn_prefill_split_rows(n) * (attn::kDim + 2) * sizeof(float);
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
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kRescaleSlack = 8.0f;  // log2 units: numerators stay <= 2^8 between rescales

// K tiles in the first 48 KiB, V tiles in the next 48 KiB, so every operand address is a per-lane
// base plus a compile-time offset below 64 KiB (the ring slot is folded into the offset).
constexpr unsigned kVBase = kStages * kTileBytes;
// 1 KiB alignment keeps the base clear of the address bits the swizzle XORs (4-8).
// After the ring: each wave's Q^T B operands of its second row block (16 k-steps x 64 lanes x
// 16 bytes), read from LDS per tile instead of occupying 64 more VGPRs.
constexpr unsigned kQ1Bytes = 16 * 64 * 16;
struct alignas(1024) Shared {
  unsigned char kv[2 * kStages * kTileBytes];
  unsigned char q1[4][kQ1Bytes];
};

// 16-byte chunk c of tile row r lives at chunk position c ^ s(r) of that row (64 banks of 4 bytes
// = 16 chunk positions; an XOR, so its own inverse):
//   K: s(r) = r % 16. The S^T operand read (ds_read_b128) of 16 consecutive lanes takes one chunk
//      of 16 consecutive rows: 16 distinct positions mod 16, no bank conflict.
//   V: s(r) = 4 (r % 4) + 16 ((r / 8) % 2). A transpose read (ds_read_b64_tr_b16) of 32 lanes
//      takes chunks 4 b .. 4 b + 3 of 4 consecutive rows 4 k .. 4 k + 3: positions
//      4 (b ^ (r % 4)) + chunk % 4, again 16 distinct. Rows r and r + 8 differ only in bit 4 of
//      the position (byte 256), rows r and r + 16 not at all.
__device__ inline unsigned swz_k(unsigned row, unsigned chunk) { return chunk ^ (row & 15u); }
__device__ inline unsigned swz_v(unsigned row, unsigned chunk) {
  return chunk ^ (4 * (row & 3u) + 16 * ((row >> 3) & 1u));
}

// Global -> LDS copy of tile rows [8 w, 8 w + 8) of K and V (one 1 KiB instruction per row pair
// and tensor). Instruction i moves tile rows 8 w + 2 i + lane / 32, chunk swz_k / swz_v(row,
// lane % 32), to LDS bytes k_lds / v_lds + 1024 i + 16 lane; its offset field (1024 i) shifts the
// global and the LDS address alike, so one M0 value serves the four instructions of a tensor and
// `koff[i]` / `voff[i]` are the lane's byte offsets inside the tile minus 1024 i. kt / vt are the
// tile's first rows (wave-uniform), so the copy needs no per-tile address arithmetic. M0 is saved
// and restored.
__device__ __attribute__((always_inline)) inline void copy_tile(const void* kt, const void* vt,
                                                                const unsigned (&koff)[4],
                                                                const unsigned (&voff)[4],
                                                                unsigned k_lds, unsigned v_lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %11\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %9\n\t"
      "global_load_lds_dwordx4 %2, %9 offset:1024\n\t"
      "global_load_lds_dwordx4 %3, %9 offset:2048\n\t"
      "global_load_lds_dwordx4 %4, %9 offset:3072\n\t"
      "s_mov_b32 m0, %12\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %5, %10\n\t"
      "global_load_lds_dwordx4 %6, %10 offset:1024\n\t"
      "global_load_lds_dwordx4 %7, %10 offset:2048\n\t"
      "global_load_lds_dwordx4 %8, %10 offset:3072\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(koff[0]), "v"(koff[1]), "v"(koff[2]), "v"(koff[3]), "v"(voff[0]), "v"(voff[1]),
        "v"(voff[2]), "v"(voff[3]), "s"(kt), "s"(vt), "s"(k_lds), "s"(v_lds)
      : "memory");
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
    const std::size_t at = std::size_t{r} * attn::kDim;
    cdna4::lds_load16(K + at + swz_k(row, lane & 31u) * 8, k_lds + m * 1024);
    cdna4::lds_load16(V + at + swz_v(row, lane & 31u) * 8, v_lds + m * 1024);
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

// One instruction of copy_tile, issued on its own so a tile's copy can be spread between MFMAs:
// instruction i (< 4: K row pair i of this wave's 8 rows, else V row pair i - 4), lane offset
// `off` from the tile's first row `row0`, to LDS byte `lds` + 1024 (i % 4) + 16 lane. M0 is
// saved and restored.
template <unsigned kI>
__device__ __attribute__((always_inline)) inline void copy_one(const void* row0, unsigned off,
                                                               unsigned lds) {
  static_assert(kI < 8, "eight instructions per wave and tile");
  unsigned saved;
  if constexpr (kI % 4 == 0)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(off), "s"(row0), "s"(lds) : "memory");
  else if constexpr (kI % 4 == 1)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2 offset:1024\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(off), "s"(row0), "s"(lds) : "memory");
  else if constexpr (kI % 4 == 2)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2 offset:2048\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(off), "s"(row0), "s"(lds) : "memory");
  else
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
                 "global_load_lds_dwordx4 %1, %2 offset:3072\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved) : "v"(off), "s"(row0), "s"(lds) : "memory");
}

// Where a tile copy goes: the tile's first K and V rows (wave-uniform), this wave's 4 KiB of the
// K and V slots, and the lane's offsets (copy_tile's koff / voff).
struct TileCopy {
  const attn::half_t* kt;
  const attn::half_t* vt;
  unsigned k_lds, v_lds;
};

// Per-lane state of one wave: two MFMA column blocks of 32 query rows (block c: tokens
// 4 c .. 4 c + 3 of the wave's 8, row n = token n / 8, head n % 8; the lane holds row col =
// lane % 32 of each). q0: block 0's Q^T B operands, dims 16 s + 8 hi + j of the lane's row,
// x log2(e)/16 (block 1's are in LDS at q1 + 1024 s + 16 lane). m[c]: the reference max in log2
// units (-inf before the first tile); l[c]: the lane half's share of the running sum.
struct Rows2 {
  half8_t q0[16];
  unsigned q1;
  float m[2], l[2];
};

// A decided tile of both blocks: its numerators as P^T B operands, [block][key step]; k-slot
// 8 hi + j of key step k holds key 16 k + 4 hi + (j < 4 ? j : j + 4) of the tile, which is how
// the S^T accumulator elements lie in the lane.
struct Numer {
  half8_t p[2][2];
};

// max(a, b, c) in one instruction (the scores are never NaN; no canonicalisation is needed).
__device__ __attribute__((always_inline)) inline float max3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// The value of x, opaque to the optimiser: address bases laundered this way stay one register,
// so the constant parts of each address fold into the LDS instructions' offsets instead of
// being re-added per access.
__device__ __attribute__((always_inline)) inline unsigned opaque(unsigned x) {
  asm volatile("" : "+v"(x));
  return x;
}

// o *= c for accumulators that live in AGPRs, element by element in place (read to a VGPR,
// multiply, write back). Written as assembly so the AGPR -> VGPR copies stay inside the caller's
// (rarely taken) branch: plain C++ lets the compiler hoist all 128 copies to the loop head. The
// leading no-ops cover the wait states between an MFMA writing o and a VALU read of it.
__device__ __attribute__((always_inline)) inline void scale_acc(float16_t (&o)[8], float c) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
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

// Softmax decision for one block of one tile. `acc`: the block's S^T accumulator (raw scores in
// log2 units; element r = key k0 + 8 (r / 4) + 4 hi + r % 4, the lane's row). Keys past `lim` are
// masked when kMasked. The reference max m moves only when the tile's row max exceeds it by more
// than the slack (2^8), decided wave-wide so the rescale branch is uniform; on the first tile (m =
// -inf) it always moves. Writes the f16 numerators 2^(s - m) as the block's two P^T operands,
// updates l = l corr + their sum (the sum of the rounded values the MFMAs use), and returns
// corr = 2^(m_old - m_new), the factor the block's O must be scaled by (1 if m stayed; `moved`
// says whether any lane's m moved).
template <bool kMasked>
__device__ __attribute__((always_inline)) inline float decide_block(const float16_t& acc,
                                                                   float& m, float& l,
                                                                   half8_t (&pb)[2], unsigned k0,
                                                                   unsigned lim, unsigned hi,
                                                                   bool& moved) {
  float x[16];
#pragma unroll
  for (unsigned r = 0; r < 16; ++r) {
    x[r] = acc[r];
    if (kMasked) {
      const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
      x[r] = key <= lim ? x[r] : -__builtin_inff();
    }
  }
  float run = max3(x[0], x[1], x[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2)
    run = max3(run, x[r], x[r + 1]);
  const float mx = cdna4::max_xor32(fmaxf(run, x[15]));
  moved = __builtin_amdgcn_ballot_w64(mx > m + kRescaleSlack) != 0;
  float corr = 1.0f;
  if (moved) {
    const float mn = fmaxf(m, mx);
    corr = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first tile (m = -inf)
    m = mn;
  }
  const cdna4::half2_t ones{static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  cdna4::half2_t e2[8];
  float lsum = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    e2[j] = cdna4::half2_t{static_cast<_Float16>(__builtin_amdgcn_exp2f(x[2 * j] - m)),
                           static_cast<_Float16>(__builtin_amdgcn_exp2f(x[2 * j + 1] - m))};
    lsum = __builtin_amdgcn_fdot2(e2[j], ones, lsum, false);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h)
    pb[h] = half8_t{e2[4 * h][0],     e2[4 * h][1],     e2[4 * h + 1][0], e2[4 * h + 1][1],
                    e2[4 * h + 2][0], e2[4 * h + 2][1], e2[4 * h + 3][0], e2[4 * h + 3][1]};
  l = l * corr + lsum;
  return corr;
}

// o += a b on the MFMA unit with the accumulator in AGPRs. Written as assembly so that O holds
// the AGPR file and the score accumulators (builtin MFMAs) stay in VGPRs, where the softmax reads
// them. The accumulator input is the output (exactly overlapping, which the hardware chains
// without wait states); every VALU access to o goes through scale_acc or the epilogue, both
// behind explicit wait states, and the B operands are rewritten only after drain_pv().
__device__ __attribute__((always_inline)) inline void pv_mfma(float16_t& o, const half8_t& a,
                                                             const half8_t& b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(o) : "v"(a), "v"(b));
}

// s = a b (first k-step, zero accumulator input) and s += a b on the MFMA unit with the score
// accumulator in VGPRs; the early-clobber output keeps the destination apart from the operands.
__device__ __attribute__((always_inline)) inline void s_mfma_first(float16_t& s, const half8_t& a,
                                                                  const half8_t& b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(s) : "v"(a), "v"(b));
}
__device__ __attribute__((always_inline)) inline void s_mfma(float16_t& s, const half8_t& a,
                                                            const half8_t& b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(s) : "v"(a), "v"(b));
}

// Wait states after an MFMA before a VALU reads its result or writes its operand registers (more
// than the 8-pass MFMA's 10). The MFMAs are assembly, so the compiler does not insert them.
__device__ __attribute__((always_inline)) inline void drain_pv() {
  asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");
}

// drain_pv's wait states tied to the score registers: an asm statement without operands orders
// only memory accesses, so the scheduler could move the softmax's VALU reads of the scores above
// it. As an in-out operand, every later use of `s` waits for the nops by data dependence.
__device__ __attribute__((always_inline)) inline void drain_scores(float16_t& s) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(s));
}

// S^T = K Q^T of one tile for both blocks: 16 k-steps over head_dim, each K operand read once
// for two MFMAs. kb: the lane's operand address in the tile's slot before the per-step XOR.
template <int kBlocks>
__device__ __attribute__((always_inline)) inline void scores2(const Rows2& rw, unsigned kb,
                                                             float16_t (&s)[kBlocks]) {
  kb = opaque(kb);  // the 16 swizzled addresses are formed at their reads, not kept live
#pragma unroll
  for (unsigned st = 0; st < 16; ++st) {
    const half8_t ka = lds_read_b128(kb ^ (32u * st));
    if (st == 0)
      s_mfma_first(s[0], ka, rw.q0[0]);
    else
      s_mfma(s[0], ka, rw.q0[st]);
    if constexpr (kBlocks == 2) {
      const half8_t q1 = lds_read_b128(rw.q1 + 1024u * st);
      if (st == 0)
        s_mfma_first(s[1], ka, q1);
      else
        s_mfma(s[1], ka, q1);
    }
  }
  drain_scores(s[0]);  // the scores are read by the softmax next
  if constexpr (kBlocks == 2)
    asm volatile("" : "+v"(s[1]));  // the nops above already cover block 1's last MFMA
}

// One tile ti of a wave, software-pipelined over two groups of MFMAs (scheduling barriers keep
// the interleave):
//   A: S^T(ti + 1) of both blocks (16 kBlocks MFMAs; each K operand read once for all blocks)
//      and the copy of tile ti + 2 (do_copy) spread one instruction per two k-steps;
//   B: O += V^T(ti) P^T(ti) (16 kBlocks MFMAs: 8 dimension blocks x 2 key steps per block, each
//      V^T operand read once for all blocks) with the decisions and numerators of tile ti + 1
//      (kNext; masked when kMaskNext) into `cur`, their VALU work spread between the MFMAs.
// The softmax VALU work needs all of S^T(ti + 1), so it can only overlap the P V MFMAs; with all
// of them in group B it has 16 kBlocks MFMAs to hide behind instead of half of them.
// A block whose m moved for tile ti + 1 has its O (holding every tile <= ti) rescaled at the end.
// kb: K operand address in slot 0, k_off the byte offset of tile ti + 1's slot; vb[c] + v_off:
// the V^T transpose-read address of 32-dim block c (rows 0-7 of key step 0) in tile ti's slot.
// Block b + 4 lies 256 bytes above block b and rows 8-15 4096 +- 256 bytes above rows 0-7, so four
// lane bases serve all 32 reads (the rest are instruction offsets).
template <int kBlocks, bool kMaskNext, bool kNext>
__device__ __attribute__((always_inline)) inline void tile_step2(
    Numer& cur, Rows2& rw, float16_t (&o)[kBlocks][8], unsigned kb, unsigned k_off,
    const unsigned (&vb)[4], unsigned v_off, unsigned k0_next, const unsigned (&lim)[2],
    unsigned hi, bool do_copy, const TileCopy& cp, const unsigned (&koff)[4],
    const unsigned (&voff)[4]) {
  // Wait states between VALU writes of this step's MFMA operands -- the numerators (written by
  // the previous decision and moved into `cur`), O (zeroed, or rescaled by scale_acc) -- and the
  // first MFMA reading them; the MFMAs are assembly, so the compiler does not insert them.
  asm volatile("s_nop 4" ::: "memory");
  const unsigned ks = kb + k_off;  // k_off has no bits below 14: the XORs below commute with it
  unsigned vt[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    vt[c] = opaque(vb[c] + v_off);
  half8_t ka[16], qa[16];
  float16_t s[kBlocks];
  auto kread = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext && st < 16) {
      ka[st] = lds_read_b128(ks ^ (32u * st));
      if (kBlocks == 2)
        qa[st] = lds_read_b128(rw.q1 + 1024u * st);
    }
  };
  auto smma = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext) {
      if (st == 0) {
        s_mfma_first(s[0], ka[0], rw.q0[0]);
        if constexpr (kBlocks == 2)
          s_mfma_first(s[1], ka[0], qa[0]);
      } else {
        s_mfma(s[0], ka[st], rw.q0[st]);
        if constexpr (kBlocks == 2)
          s_mfma(s[1], ka[st], qa[st]);
      }
    }
  };
  // V^T operands in MFMA order (dimension blocks 0-7 of key step 0, then of key step 1), each
  // used by both row blocks, three ahead.
  constexpr unsigned kAhead = 3;
  half8_t va[kAhead];
  auto vread = [&](unsigned i) __attribute__((always_inline)) {
    if (i < 16) {
      const unsigned b = i % 8, step = i / 8;
      const unsigned at = vt[b % 4] + 256u * (b / 4) + 8192u * step;
      const half4_t lo = read_tr(at);
      const half4_t up = read_tr(at + (b < 4 ? 4096u + 256u : 4096u - 256u));
      va[i % kAhead] = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
    }
  };
  auto pv = [&](unsigned i, unsigned c) __attribute__((always_inline)) {
    const unsigned b = i % 8, step = i / 8;
    pv_mfma(o[c][b], va[i % kAhead], cur.p[c][step]);
  };
  auto copy = [&](unsigned st) __attribute__((always_inline)) {
    if (do_copy) {  // uniform
      switch (st) {
        case 1: copy_one<0>(cp.kt, koff[0], cp.k_lds); break;
        case 3: copy_one<1>(cp.kt, koff[1], cp.k_lds); break;
        case 5: copy_one<2>(cp.kt, koff[2], cp.k_lds); break;
        case 7: copy_one<3>(cp.kt, koff[3], cp.k_lds); break;
        case 9: copy_one<4>(cp.vt, voff[0], cp.v_lds); break;
        case 11: copy_one<5>(cp.vt, voff[1], cp.v_lds); break;
        case 13: copy_one<6>(cp.vt, voff[2], cp.v_lds); break;
        case 15: copy_one<7>(cp.vt, voff[3], cp.v_lds); break;
        default: break;
      }
    }
  };

  // Group A: the score MFMAs, the first V^T operands read ahead for group B.
  kread(0);
  kread(1);
#pragma unroll
  for (unsigned i = 0; i < kAhead; ++i)
    vread(i);
#pragma unroll
  for (unsigned st = 0; st < 16; ++st) {
    kread(st + 2);
    smma(st);
    copy(st);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Group B: the decisions of tile ti + 1 (the arithmetic of decide_block, in the same order),
  // cut into items spread over the slots so the VALU work issues between the MFMAs. Per block c:
  // X (mask, first half of the row max) and Y (row max, wave-wide move decision, new reference
  // max); per numerator pair k (pairs alternate between the blocks) two SE halves (a difference
  // and its 2^x each) and CD (the f16 pair and its share of the row sum); F (operands, l) at the
  // end. Each result is pinned by an empty volatile asm where it is made: the numerators are
  // used only at the end of the step, and the compiler would otherwise sink their arithmetic
  // below the last MFMA, where it runs with the matrix unit idle.
  bool moved[2] = {false, false};
  float corr[2] = {1.0f, 1.0f};
  float x[kBlocks][16], run[kBlocks], lsum[kBlocks], ex[kBlocks][16];
  cdna4::half2_t e2[kBlocks][8];
  half8_t next[2][2];
  const cdna4::half2_t ones{static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  auto stage_x = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (unsigned r = 0; r < 16; ++r) {
      x[c][r] = s[c][r];
      if (kMaskNext) {
        const unsigned key = k0_next + 8 * (r / 4) + 4 * hi + (r % 4);
        x[c][r] = key <= lim[c] ? x[c][r] : -__builtin_inff();
      }
    }
    run[c] = max3(x[c][0], x[c][1], x[c][2]);
    run[c] = max3(run[c], x[c][3], x[c][4]);
    run[c] = max3(run[c], x[c][5], x[c][6]);
    run[c] = max3(run[c], x[c][7], x[c][8]);
    asm volatile("" : "+v"(run[c]));
  };
  auto stage_y = [&](int c) __attribute__((always_inline)) {
    run[c] = max3(run[c], x[c][9], x[c][10]);
    run[c] = max3(run[c], x[c][11], x[c][12]);
    run[c] = max3(run[c], x[c][13], x[c][14]);
    const float mx = cdna4::max_xor32(fmaxf(run[c], x[c][15]));
    moved[c] = __builtin_amdgcn_ballot_w64(mx > rw.m[c] + kRescaleSlack) != 0;
    if (moved[c]) {
      const float mn = fmaxf(rw.m[c], mx);
      corr[c] = __builtin_amdgcn_exp2f(rw.m[c] - mn);  // 0 on the first tile (m = -inf)
      rw.m[c] = mn;
    }
    asm volatile("" : "+v"(rw.m[c]));
  };
  // Numerator pair k: block k % kBlocks, pair j = k / kBlocks (keys 2 j, 2 j + 1 of the lane).
  auto stage_se = [&](unsigned k, unsigned half) __attribute__((always_inline)) {
    const int c = static_cast<int>(k % kBlocks);
    const unsigned r = 2 * (k / kBlocks) + half;
    ex[c][r] = __builtin_amdgcn_exp2f(x[c][r] - rw.m[c]);
    asm volatile("" : "+v"(ex[c][r]));
  };
  auto stage_cd = [&](unsigned k) __attribute__((always_inline)) {
    const int c = static_cast<int>(k % kBlocks);
    const unsigned j = k / kBlocks;
    e2[c][j] = cdna4::half2_t{static_cast<_Float16>(ex[c][2 * j]),
                              static_cast<_Float16>(ex[c][2 * j + 1])};
    lsum[c] = __builtin_amdgcn_fdot2(e2[c][j], ones, j == 0 ? 0.0f : lsum[c], false);
    asm volatile("" : "+v"(e2[c][j]), "+v"(lsum[c]));
  };
  auto stage_f = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      next[c][h] = half8_t{e2[c][4 * h][0],     e2[c][4 * h][1],     e2[c][4 * h + 1][0],
                           e2[c][4 * h + 1][1], e2[c][4 * h + 2][0], e2[c][4 * h + 2][1],
                           e2[c][4 * h + 3][0], e2[c][4 * h + 3][1]};
    rw.l[c] = rw.l[c] * corr[c] + lsum[c];
  };
  // Work items in order: X of each block, Y of each block, then per numerator pair k its two
  // halves of SE (one difference and its 2^x each) with the CD of pair k - 1 after them, then
  // the last CD and F. Item n runs in slot n kSlots / kItems: an even spread, and a pair's CD
  // lands about two slots after its SE, so no slot waits on a result it made itself.
  constexpr unsigned kSlots = 16 * kBlocks;  // one P V MFMA each
  constexpr unsigned kPairs = 8 * kBlocks;
  constexpr unsigned kBase = 2 * kBlocks;
  constexpr unsigned kItems = kBase + 3 * kPairs + 2;
  auto item = [&](unsigned n) __attribute__((always_inline)) {
    if (n < kBlocks) {
      stage_x(static_cast<int>(n));
    } else if (n < kBase) {
      stage_y(static_cast<int>(n - kBlocks));
    } else if (n < kBase + 3 * kPairs) {
      const unsigned k = (n - kBase) / 3, part = (n - kBase) % 3;
      if (part < 2)
        stage_se(k, part);
      else if (k > 0)
        stage_cd(k - 1);
    } else if (n == kBase + 3 * kPairs) {
      stage_cd(kPairs - 1);
    } else {
#pragma unroll
      for (int b = 0; b < kBlocks; ++b)
        stage_f(b);
    }
  };
#pragma unroll
  for (unsigned q = 0; q < kSlots; ++q) {
    // P V MFMAs in issue order: operand i (dimension block i % 8 of key step i / 8) for blocks
    // 0 .. kBlocks - 1, each operand read once for all blocks.
    const unsigned i = q / kBlocks;
    const int c = static_cast<int>(q % kBlocks);
    pv(i, c);
    if (c == kBlocks - 1)
      vread(i + kAhead);
    if (kNext) {
      if (q == 0) {
        // The last score MFMA is at least one MFMA back; its results are read next.
        drain_scores(s[0]);
        if constexpr (kBlocks == 2)
          asm volatile("" : "+v"(s[1]));
      }
      const unsigned first = (q * kItems + kSlots - 1) / kSlots;
      const unsigned end = ((q + 1) * kItems + kSlots - 1) / kSlots;
#pragma unroll
      for (unsigned n = first; n < end; ++n)
        item(n);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  drain_pv();
  if (kNext) {
#pragma unroll
    for (int c = 0; c < kBlocks; ++c)
      cur.p[c][0] = next[c][0], cur.p[c][1] = next[c][1];
#pragma unroll
    for (int c = 0; c < kBlocks; ++c)
      if (moved[c])
        scale_acc(o[c], corr[c]);
  }
}

}  // namespace prefill_detail

// Items [first, first + count) (grid-stride). Item -> (KV head, token block) as described at
// attn_prefill_items. Per workgroup: 16 kBlocks tokens x 8 heads of one KV head; wave w owns
// 4 kBlocks of them, kBlocks MFMA column blocks of 4 tokens x 8 heads (row n of a block = token
// offset n / 8, head n % 8).
//
// K/V tiles of 32 keys stream into a 3-stage LDS ring by direct global->LDS loads (each wave
// copies 8 rows of each, one instruction at a time between its MFMAs); one barrier per tile. Per
// tile i (tile_step2): S^T(i + 1) = K Q^T (16 MFMAs per block; the first block's Q^T resident in
// VGPRs as f16 pre-scaled by log2(e)/16, the second's in LDS), then O^T += V^T P^T(i) for every
// block (16 MFMAs per block, V^T from ds_read_b64_tr_b16, each operand feeding every block) with
// the decisions and numerators of tile i + 1 issued between those MFMAs. Keys past a row's causal
// limit are masked only in the diagonal tiles of a wave; the gate and 1/l are applied at the
// store.
namespace prefill_detail {

// A workgroup's run over one token block: tiles [tb, te) of its keys; `part` says the tiles are
// one of two parts of a split block (partial to workspace slot `slot`, merge by the later part).
struct PrefillJob {
  unsigned kvh, blk, tb, te, slot;
  bool part;
};

// Tiles of keys block b of kTokens tokens sees (its last token's causal limit).
template <unsigned kTokens>
__device__ __attribute__((always_inline)) inline unsigned block_tiles(const AttnPrefillParams& p,
                                                                      unsigned b) {
  return (p.pos0 + min((b + 1) * kTokens, p.n) + kKeys - 1) / kKeys;
}

// The jobs of item `item` (wave-uniform): one for the one-block-per-workgroup layout of
// attn_prefill_items, up to two for the balanced layout of attn_prefill_split_items.
template <unsigned kTokens, bool kSplit>
__device__ __attribute__((always_inline)) inline unsigned item_jobs(const AttnPrefillParams& p,
                                                                    unsigned item,
                                                                    unsigned blocks,
                                                                    PrefillJob (&jobs)[2]) {
  const unsigned xcd = item % 8, kvh = xcd / 4;
  if constexpr (!kSplit) {
    const unsigned rank = (item / 8) * 4 + xcd % 4;
    if (rank >= blocks)
      return 0;
    const unsigned blk = blocks - 1 - rank;
    jobs[0] = PrefillJob{kvh, blk, 0, block_tiles<kTokens>(p, blk), 0, false};
    return 1;
  } else {
    const unsigned role = (item / 8) % 2, pair = (item / 16) * 4 + xcd % 4;
    const unsigned pairs = blocks / 2;
    if (pair >= pairs) {  // the middle block of an odd count (workgroup A), or nothing
      if (pair > pairs || blocks % 2 == 0 || role == 1)
        return 0;
      jobs[0] = PrefillJob{kvh, pair, 0, block_tiles<kTokens>(p, pair), 0, false};
      return 1;
    }
    const unsigned hb = blocks - 1 - pair, lb = pair;
    const unsigned th = block_tiles<kTokens>(p, hb), tl = block_tiles<kTokens>(p, lb);
    const unsigned bias = kTokens == kAttnQBlock ? kAttnSplitBias : kAttnSplitBias2;
    const unsigned cut = (th + tl + 1) / 2 + bias;
    // Tiles every row of the heavy block sees in full: the split point stays among them.
    const unsigned full = (p.pos0 + hb * kTokens + 1) / kKeys;
    if (cut + kAttnSplitMinTiles > th || cut > full) {
      jobs[0] = role == 0 ? PrefillJob{kvh, hb, 0, th, 0, false}
                          : PrefillJob{kvh, lb, 0, tl, 0, false};
      return 1;
    }
    const unsigned slot = 2 * (kvh * pairs + pair) + role;
    if (role == 0) {
      jobs[0] = PrefillJob{kvh, hb, 0, cut, slot, true};
      return 1;
    }
    jobs[0] = PrefillJob{kvh, hb, cut, th, slot, true};
    jobs[1] = PrefillJob{kvh, lb, 0, tl, 0, false};
    return 2;
  }
}

template <int kBlocks, bool kSplit = false>
__device__ __attribute__((always_inline)) inline void prefill_items(
    const AttnPrefillParams& p, const AttnPrefillSplitParams* sp, unsigned first, unsigned count,
    Shared& sh) {
  using attn::kDim;
  constexpr int kGroup = attn::kQHeads / attn::kKvHeads;
  constexpr unsigned kItemTokens = kAttnQBlock * kBlocks;
  constexpr unsigned kWaveTokens = kItemTokens / 4;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned col = lane & 31u, hi = lane >> 5;  // MFMA column / lane half
  const unsigned blocks = (p.n + kItemTokens - 1) / kItemTokens;
  const unsigned lds0 = cdna4::lds_offset(sh.kv);

  // Per-lane constant addresses. Copy: instruction i moves rows 8 w + 2 i + lane / 32 (its
  // offset field adds the 1024 i).
  unsigned copy_koff[4], copy_voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const unsigned row = 8 * wave + 2 * i + (lane >> 5);
    copy_koff[i] = row * kRowBytes + swz_k(row, lane & 31u) * 16 - 1024 * i;
    copy_voff[i] = row * kRowBytes + swz_v(row, lane & 31u) * 16 - 1024 * i;
  }
  // S^T A operand (key row col, chunk 2 st + hi at position (2 st + hi) ^ (col % 16)):
  // (col 512 + 16 (hi ^ (col % 16))) ^ 32 st.
  const unsigned kb = lds0 + col * kRowBytes + 16 * (hi ^ (col & 15u));
  // V^T transpose reads: rows 16 step + vrow (+ 8), chunk 4 b + vchunk, byte vbyte, i.e.
  // (512 vrow + vbyte + 16 vchunk + 64 (vrow % 4)) ^ (64 b) [^ 256, + 4096 for rows + 8]
  // + 8192 step. Bit 8 of the part before the XOR is clear, so blocks 4-7 are blocks 0-3 + 256 and
  // the rows + 8 are + 4096 -+ 256: vb[c] (block c, rows 0-7, slot 0) is all a lane needs.
  unsigned vb[4];
  {
    const unsigned g = lane >> 4, j = lane & 15u;
    const unsigned vrow = 4 * (g >> 1) + j / 4, vchunk = 2 * (g & 1u) + (j % 4) / 2;
    const unsigned vbyte = 8 * ((j % 4) & 1u);
    const unsigned base = vrow * kRowBytes + vbyte + 16 * swz_v(vrow, vchunk);
#pragma unroll
    for (int c = 0; c < 4; ++c)
      vb[c] = lds0 + kVBase + (base ^ (64u * c));
  }

  for (unsigned item = first + blockIdx.x; item < first + count; item += gridDim.x) {
    PrefillJob jobs[2];
    const unsigned njobs = item_jobs<kItemTokens, kSplit>(p, item, blocks, jobs);
    for (unsigned j = 0; j < njobs; ++j) {  // uniform across the workgroup
      const PrefillJob jb = j == 0 ? jobs[0] : jobs[1];
      const unsigned kvh = jb.kvh, blk = jb.blk, tb = jb.tb;
      const unsigned t0 = blk * kItemTokens;
      const unsigned t_end = min(t0 + kItemTokens, p.n);
      const unsigned kv_end = p.pos0 + t_end;
      const attn::half_t* K = p.k_cache + std::size_t{kvh} * p.max_ctx * kDim;
      const attn::half_t* V = p.v_cache + std::size_t{kvh} * p.max_ctx * kDim;
      const unsigned tiles = jb.te;  // this job's tiles: [tb, tiles)
      // Ring slots as byte offsets, rotated once per tile: tile ti is in `cur`, ti + 1 in `next`,
      // ti + 2 goes to `spare`.
      unsigned slot_cur = 0, slot_next = kTileBytes, slot_spare = 2 * kTileBytes;
      auto rotate = [&]() __attribute__((always_inline)) {
        const unsigned tmp = slot_cur;
        slot_cur = slot_next;
        slot_next = slot_spare;
        slot_spare = tmp;
      };
      auto full_tile = [&](unsigned ti) __attribute__((always_inline)) {
        return (ti + 1) * kKeys <= kv_end;
      };
      auto dest = [&](unsigned ti, unsigned slot) __attribute__((always_inline)) {
        return TileCopy{K + std::size_t{ti} * kKeys * kDim, V + std::size_t{ti} * kKeys * kDim,
                        lds0 + slot + wave * 4096, lds0 + kVBase + slot + wave * 4096};
      };
      // A whole tile copy at once (the first two tiles, and the last one when it crosses kv_end).
      auto copy = [&](unsigned ti, unsigned slot) __attribute__((always_inline)) {
        const TileCopy d = dest(ti, slot);
        if (full_tile(ti))
          copy_tile(d.kt, d.vt, copy_koff, copy_voff, d.k_lds, d.v_lds);
        else
          copy_tile_clamped(K, V, ti * kKeys, kv_end - 1, d.k_lds - wave * 4096,
                            d.v_lds - wave * 4096, wave, lane);
      };

      // Start streaming before anything else: the job's first two tiles.
      copy(tb, slot_cur);
      if (tiles > tb + 1)
        copy(tb + 1, slot_next);

      // This wave's rows: block c, token tw + 4 c + col / 8, head kvh * 8 + col % 8.
      const unsigned tw = t0 + kWaveTokens * wave, hq = col % kGroup;
      unsigned tq[2] = {0, 0}, lim[2] = {0, 0};
      bool q_valid[2] = {false, false};
#pragma unroll
      for (int c = 0; c < kBlocks; ++c) {
        const unsigned raw_t = tw + 4 * c + col / kGroup;
        q_valid[c] = raw_t < p.n;
        tq[c] = q_valid[c] ? raw_t : p.n - 1;
        lim[c] = p.pos0 + tq[c];  // last visible key
      }
      const bool wave_active = tw < p.n;
      // Tiles this wave needs, and how many of them every row of the wave sees in full (always
      // fewer: the last tile of a wave is a diagonal one).
      const unsigned wave_tiles =
          wave_active ? (p.pos0 + min(tw + kWaveTokens - 1, p.n - 1)) / kKeys + 1 : 0;
      const unsigned full_tiles = wave_active ? (p.pos0 + tw + 1) / kKeys : 0;

      Rows2 rw;
      rw.q1 = cdna4::lds_offset(sh.q1[wave]) + 16 * lane;
      constexpr float kScale = kLog2e / 16.0f;  // 1/sqrt(256) in log2 units
      if constexpr (kBlocks == 1) {
        // Q^T B operands: lane (col, hi) needs row col, one row per lane, which as global loads
        // would take the address unit one lane per cycle. Instead each load moves one row (1 KiB,
        // lane l: dimensions 4 l .. 4 l + 3), the f16 rows go to this wave's Q^T area (unused
        // with one block: 32 rows x 512 bytes, 16-byte chunk c of row r at position c ^ (r % 16),
        // so the writes of a row and the reads of 16 rows at one chunk hit distinct banks), and
        // each lane reads its operands back. Rows of tokens >= n are zero (they are not stored).
        const unsigned qa = cdna4::lds_offset(sh.q1[wave]);
        float4 x[32];
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const unsigned tk = min(tw + r / 8, p.n - 1);
          x[r] = *reinterpret_cast<const float4*>(
              p.q + (std::size_t{tk} * attn::kQHeads + kvh * kGroup + r % 8) * kDim + 4 * lane);
        }
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const float z = tw + r / 8 < p.n ? kScale : 0.0f;
          const half4_t h = {static_cast<_Float16>(x[r].x * z), static_cast<_Float16>(x[r].y * z),
                             static_cast<_Float16>(x[r].z * z), static_cast<_Float16>(x[r].w * z)};
          *reinterpret_cast<__attribute__((address_space(3))) half4_t*>(
              qa + 512 * r + 16 * ((lane / 2) ^ (r & 15)) + 8 * (lane & 1)) = h;
        }
#pragma unroll
        for (int st = 0; st < 16; ++st)
          rw.q0[st] = *reinterpret_cast<const __attribute__((address_space(3))) half8_t*>(
              qa + 512 * col + 16 * ((2 * st + hi) ^ (col & 15)));
        rw.m[0] = -__builtin_inff();
        rw.l[0] = 0.0f;
      } else {
#pragma unroll
        for (int c = 0; c < kBlocks; ++c) {
          const float* src =
              p.q + (std::size_t{tq[c]} * attn::kQHeads + kvh * kGroup + hq) * kDim + 8 * hi;
          const float z = q_valid[c] ? kScale : 0.0f;
#pragma unroll
          for (int st = 0; st < 16; ++st) {
            const float4 x0 = *reinterpret_cast<const float4*>(src + 16 * st);
            const float4 x1 = *reinterpret_cast<const float4*>(src + 16 * st + 4);
            const half8_t v =
                half8_t{static_cast<_Float16>(x0.x * z), static_cast<_Float16>(x0.y * z),
                        static_cast<_Float16>(x0.z * z), static_cast<_Float16>(x0.w * z),
                        static_cast<_Float16>(x1.x * z), static_cast<_Float16>(x1.y * z),
                        static_cast<_Float16>(x1.z * z), static_cast<_Float16>(x1.w * z)};
            if (c == 0)
              rw.q0[st] = v;
            else  // this wave's own region: its later reads are ordered after these writes
              *reinterpret_cast<__attribute__((address_space(3))) half8_t*>(rw.q1 + 1024u * st) =
                  v;
          }
          rw.m[c] = -__builtin_inff();
          rw.l[c] = 0.0f;
        }
      }
      float16_t oacc[kBlocks][8];
#pragma unroll
      for (int c = 0; c < kBlocks; ++c)
#pragma unroll
        for (int b = 0; b < 8; ++b)
          oacc[c][b] = float16_t{};

      // Start of iteration ti: tile ti + 1 complete in LDS -- this wave's share by vmcnt (its
      // copy was the last one issued), every wave's by the barrier, which also says that all waves
      // are done with tile ti - 1, whose slot then receives tile ti + 2 during the step.
      auto sync = [&](unsigned ti) __attribute__((always_inline)) {
        if (ti + 1 < tiles) {
          cdna4::wait_vmcnt<0>();
          __syncthreads();
        }
      };
      // The step's copy of tile ti + 2: spread inside the step for a full tile, else at once.
      auto next_copy = [&](unsigned ti) __attribute__((always_inline)) {
        const bool spread = ti + 2 < tiles && full_tile(ti + 2);
        if (ti + 2 < tiles && !spread)
          copy(ti + 2, slot_spare);
        return spread;
      };

      cdna4::wait_vmcnt<0>();  // tiles 0 (and 1) and the queries are in
      __syncthreads();
      // cur: the decided numerators of tile ti at the top of iteration ti (tile 0: here; O is
      // still 0, so the first decision needs no rescale).
      Numer cur;
      if (wave_active) {
        float16_t s0[kBlocks];
        scores2<kBlocks>(rw, kb, s0);
        bool mv;
#pragma unroll
        for (int c = 0; c < kBlocks; ++c) {
          if (full_tiles > tb)
            decide_block<false>(s0[c], rw.m[c], rw.l[c], cur.p[c], tb * kKeys, lim[c], hi, mv);
          else
            decide_block<true>(s0[c], rw.m[c], rw.l[c], cur.p[c], tb * kKeys, lim[c], hi, mv);
        }
      }
      // One pass over the workgroup's tiles in phases per wave, each a loop with a single body
      // (the per-wave bounds differ; every wave still runs sync once per tile, in order): tiles
      // whose successor the wave's rows see in full, tiles whose successor is diagonal, the last
      // tile (no successor), then the tiles the wave does not need.
      unsigned ti = tb;
      auto step = [&](auto mask_next, auto has_next) __attribute__((always_inline)) {
        sync(ti);
        const bool spread = next_copy(ti);
        tile_step2<kBlocks, decltype(mask_next)::value, decltype(has_next)::value>(
            cur, rw, oacc, kb, slot_next, vb, slot_cur, (ti + 1) * kKeys, lim, hi, spread,
            dest(ti + 2, slot_spare), copy_koff, copy_voff);
      };
      using F = std::false_type;
      using T = std::true_type;
      const unsigned full_end = min(full_tiles, tiles), wave_end = min(wave_tiles, tiles);
      for (; ti + 1 < full_end; ++ti, rotate())
        step(F{}, T{});
      for (; ti + 1 < wave_end; ++ti, rotate())
        step(T{}, T{});
      if (ti < wave_end) {
        step(F{}, F{});
        ++ti;
        rotate();
      }
      for (; ti < tiles; ++ti, rotate()) {
        sync(ti);
        if (ti + 2 < tiles)
          copy(ti + 2, slot_spare);
      }
      __syncthreads();  // the ring is reused by the next item
      drain_pv();

      // Output: core = O / l * sigmoid(gate). In the accumulator layout a lane holds one row
      // (its column), so a global access of a wave would touch 32 rows 1 KiB apart, 16 bytes
      // each, and the address unit handles such an access one lane per cycle. O / l therefore
      // goes through this wave's LDS (the ring and the Q^T area are free after the barrier
      // above): row r at byte kStageRow r, padded by one 16-byte chunk so the 16 lanes of a write
      // (16 rows, one chunk) and of a read (one row, 16 chunks) hit distinct banks; every address
      // is one register plus an immediate. Then each gate load and core store moves one whole
      // row (1 KiB, lane l: dimensions 4 l .. 4 l + 3).
      constexpr unsigned kStageRow = 1024 + 16;
      static_assert(4 * 32 * kStageRow <= sizeof(Shared));
      const unsigned stage = lds0 + wave * 32 * kStageRow;
      auto stage_o = [&](int c, float f) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < 8; ++b)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const unsigned k = 8 * b + 2 * r4 + hi;
            const cdna4::float4_t o = {oacc[c][b][4 * r4 + 0] * f, oacc[c][b][4 * r4 + 1] * f,
                                       oacc[c][b][4 * r4 + 2] * f, oacc[c][b][4 * r4 + 3] * f};
            *reinterpret_cast<__attribute__((address_space(3))) cdna4::float4_t*>(
                stage + kStageRow * col + 16 * k) = o;
          }
      };
      auto staged_row = [&](int r) __attribute__((always_inline)) {
        return *reinterpret_cast<const __attribute__((address_space(3))) cdna4::float4_t*>(
            stage + kStageRow * r + 16 * lane);
      };
      // Row total: each column's keys per tile were split between the lane halves.
      float l_row[kBlocks];
#pragma unroll
      for (int c = 0; c < kBlocks; ++c)
        l_row[c] = cdna4::sum_xor32(rw.l[c]);
      // A part of a split block: its partial to the workspace (rows of O relative to 2^m, and
      // (m, l) per row), then the agent-scope counter of the pair; the part that arrives second
      // merges (one that finds the counter already set merges without writing its own).
      // Merged rows: O = O_A f_A + O_B f_B, f_X = 2^(m_X - M) / (l_A 2^(m_A - M) +
      // l_B 2^(m_B - M)), M the larger m, evaluated in this order whichever part merges (the
      // output does not depend on which part arrives second).
      //
      // The partials move with agent-coherent buffer accesses (cache policy sc1, what a relaxed
      // agent-scope atomic access compiles to on gfx950): they are not left dirty in, nor read
      // stale from, an XCD's L2. Each wave waits for its partial stores to complete, the
      // barrier orders them before thread 0's counter increment, and the merging part's loads
      // are issued after it has read the count. An agent-scope release fence would instead write
      // back every dirty line of the L2 (the other workgroups' output included), which stalls
      // the XCD for microseconds.
      bool store = true, merge = false;
      float f_a[kBlocks] = {}, f_b[kBlocks] = {};  // this lane's row (column col)
      bool own_a = true;
      const float* oth = nullptr;  // the other part's rows of this wave (this lane's 16 bytes)
      constexpr int kSc1 = 16;  // cache-policy operand of the buffer builtins: sc1
      const auto part_rsrc = [&](float* base, unsigned floats) __attribute__((always_inline)) {
        return __builtin_amdgcn_make_buffer_rsrc(base, 0, static_cast<int>(4 * floats),
                                                 0x00020000);
      };
      // A part's rows: slot * kPartRows + 32 kBlocks wave + 32 c + r (block c, row r).
      constexpr unsigned kPartRows = 128 * kBlocks;
      const unsigned part_rows = 2 * attn_prefill_split_pairs(p.n) * kPartRows;
      if constexpr (kSplit) {
        if (jb.part) {
          const auto o_rsrc = part_rsrc(sp->part_o, part_rows * kDim);
          const auto ml_rsrc = part_rsrc(sp->part_ml, part_rows * 2);
          const unsigned row0 = jb.slot * kPartRows + 32 * kBlocks * wave;
          auto* flag = reinterpret_cast<__attribute__((address_space(3))) unsigned*>(
              lds0 + 4 * 32 * kStageRow);  // past every wave's staging
          unsigned* counter = sp->counters + jb.slot / 2;
          // If the other part has published already, merge without publishing this one.
          if (t == 0)
            *flag = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __syncthreads();
          store = *flag != 0;
          if (!store) {  // uniform
#pragma unroll
            for (int c = 0; c < kBlocks; ++c) {
              stage_o(c, 1.0f);
              if (hi == 0)
                __builtin_amdgcn_raw_buffer_store_b64(
                    __builtin_bit_cast(cdna4::u32x2_t, float2{rw.m[c], l_row[c]}), ml_rsrc,
                    (row0 + 32 * c + col) * 8, 0, kSc1);
#pragma unroll
              for (int r = 0; r < 32; ++r)
                __builtin_amdgcn_raw_buffer_store_b128(
                    __builtin_bit_cast(cdna4::u32x4_t, staged_row(r)), o_rsrc,
                    (row0 + 32 * c + r) * 1024 + 16 * lane, 0, kSc1);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // every wave's partial complete, and the flag read
            if (t == 0)
              *flag = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            store = *flag != 0;
          }
          if (store) {  // uniform: the other part's partial is complete
            if (t == 0)  // every launch leaves the counters zero
              __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned orow0 = (jb.slot ^ 1u) * kPartRows + 32 * kBlocks * wave;
            own_a = (jb.slot & 1u) == 0;
#pragma unroll
            for (int c = 0; c < kBlocks; ++c) {
              const float2 oml = __builtin_bit_cast(
                  float2, __builtin_amdgcn_raw_buffer_load_b64(ml_rsrc, (orow0 + 32 * c + col) * 8,
                                                               0, kSc1));
              const float m_a = own_a ? rw.m[c] : oml.x, m_b = own_a ? oml.x : rw.m[c];
              const float l_a = own_a ? l_row[c] : oml.y, l_b = own_a ? oml.y : l_row[c];
              const float m_max = fmaxf(m_a, m_b);
              const float e_a = __builtin_amdgcn_exp2f(m_a - m_max);
              const float e_b = __builtin_amdgcn_exp2f(m_b - m_max);
              const float inv_l = __builtin_amdgcn_rcpf(l_a * e_a + l_b * e_b);
              f_a[c] = e_a * inv_l;
              f_b[c] = e_b * inv_l;
            }
            merge = true;
            oth = sp->part_o + std::size_t{orow0} * kDim + 4 * lane;
          }
        }
      }
      if (store) {
#pragma unroll
        for (int c = 0; c < kBlocks; ++c) {
          if (!merge) {
            stage_o(c, __builtin_amdgcn_rcpf(l_row[c]));
          } else if constexpr (kSplit) {
            // The other part's rows of the block straight into the staging (one agent-coherent
            // LDS-DMA load per row), then each lane combines its own accumulators with them in
            // place: O_A f_A + O_B f_B for its row.
#pragma unroll
            for (int r = 0; r < 32; ++r)
              __builtin_amdgcn_global_load_lds(
                  oth + (32 * c + r) * kDim,
                  reinterpret_cast<__attribute__((address_space(3))) void*>(stage + kStageRow * r),
                  16, 0, kSc1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int b = 0; b < 8; ++b)
#pragma unroll
              for (int r4 = 0; r4 < 4; ++r4) {
                auto* at = reinterpret_cast<__attribute__((address_space(3))) cdna4::float4_t*>(
                    stage + kStageRow * col + 16 * (8 * b + 2 * r4 + hi));
                const cdna4::float4_t w = *at;
                const cdna4::float4_t v = {oacc[c][b][4 * r4 + 0], oacc[c][b][4 * r4 + 1],
                                           oacc[c][b][4 * r4 + 2], oacc[c][b][4 * r4 + 3]};
                const cdna4::float4_t oa = own_a ? v : w, ob = own_a ? w : v;
                *at = cdna4::float4_t{__builtin_fmaf(ob[0], f_b[c], oa[0] * f_a[c]),
                                      __builtin_fmaf(ob[1], f_b[c], oa[1] * f_a[c]),
                                      __builtin_fmaf(ob[2], f_b[c], oa[2] * f_a[c]),
                                      __builtin_fmaf(ob[3], f_b[c], oa[3] * f_a[c])};
              }
          }
          // Rows 8 j + h of the block: token tw + 4 c + j, head kvh * 8 + h; tokens >= n are not
          // stored (their gate loads read token n - 1).
          const unsigned tok0 = tw + 4 * c;
          const float* gate = p.qg + std::size_t{kvh} * kGroup * 2 * kDim + kDim + 4 * lane;
          float* out = p.core + std::size_t{kvh} * kGroup * kDim + 4 * lane;
          // Gate rows in flight: all 32 of the block with one block of O in the AGPRs; with two,
          // 16 at a time (the loads of the second half then wait behind the stores of the first).
          constexpr int kGateRows = kBlocks == 1 ? 32 : 16;
#pragma unroll
          for (int r0 = 0; r0 < 32; r0 += kGateRows) {
            float4 gv[kGateRows];
#pragma unroll
            for (int r = r0; r < r0 + kGateRows; ++r) {
              const unsigned tk = min(tok0 + r / 8, p.n - 1);
              gv[r - r0] = *reinterpret_cast<const float4*>(gate + std::size_t{tk} * p.qg_stride +
                                                            (r % 8) * 2 * kDim);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = r0; r < r0 + kGateRows; ++r) {
              const cdna4::float4_t v = staged_row(r);
              const float4 g = gv[r - r0];
              float4 o;
              o.x = v[0] * __builtin_amdgcn_rcpf(1.0f + __expf(-g.x));
              o.y = v[1] * __builtin_amdgcn_rcpf(1.0f + __expf(-g.y));
              o.z = v[2] * __builtin_amdgcn_rcpf(1.0f + __expf(-g.z));
              o.w = v[3] * __builtin_amdgcn_rcpf(1.0f + __expf(-g.w));
              if (tok0 + r / 8 < p.n)  // uniform
                *reinterpret_cast<float4*>(out + (std::size_t{tok0 + r / 8} * attn::kQHeads +
                                                  r % 8) * kDim) = o;
            }
          }
        }
      }
      if (j + 1 < njobs || item + gridDim.x < first + count)
        __syncthreads();  // the next job's copies overwrite the staging
    }
  }
}

}  // namespace prefill_detail

template <int kBlock>
__device__ void attn_prefill_op(const AttnPrefillParams& p, unsigned first, unsigned count) {
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  __shared__ prefill_detail::Shared sh;
  if (attn_prefill_row_blocks(p.n) == 2)  // uniform: the item size follows n
    prefill_detail::prefill_items<2>(p, nullptr, first, count, sh);
  else
    prefill_detail::prefill_items<1>(p, nullptr, first, count, sh);
}

template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prefill_kernel(AttnPrefillParams p) {
  attn_prefill_op<kBlock>(p, 0, attn_prefill_items(p.n));
}

// The balanced form (attn_prefill_split_items(n) workgroups of 256; attn_prefill_balanced(n)).
template <int kBlock>
__global__ void __launch_bounds__(kBlock) attn_prefill_split_kernel(AttnPrefillSplitParams p) {
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  __shared__ prefill_detail::Shared sh;
  const unsigned items = attn_prefill_split_items(p.a.n);
  if (attn_prefill_balanced_blocks(p.a.n) == 2)  // uniform: the block size follows n
    prefill_detail::prefill_items<2, true>(p.a, &p, 0, items, sh);
  else
    prefill_detail::prefill_items<1, true>(p.a, &p, 0, items, sh);
}

}  // namespace miso::kernels
