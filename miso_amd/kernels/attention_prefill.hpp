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

// Tokens per workgroup: 4 waves x 4 tokens; a wave's 4 tokens x 8 query heads are the 32 rows of
// one MFMA column block.
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
struct alignas(1024) Shared {
  unsigned char kv[2 * kStages * kTileBytes];
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

// Per-lane state of one wave (32 query rows = one MFMA column block): the Q^T B operands, dims
// 16 s + 8 hi + j of the lane's row, x log2(e)/16; the reference max m and running sum l; and -m
// in all 16 elements, the initial S^T accumulator, so the scores come out of the MFMAs relative
// to m.
struct Rows {
  half8_t q[16];
  float m, l;
  float16_t negm;
};

__device__ __attribute__((always_inline)) inline float16_t splat16(float x) {
  float16_t v;
#pragma unroll
  for (int r = 0; r < 16; ++r)
    v[r] = x;
  return v;
}

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

// S^T[key][row] = K Q^T for one tile (32 keys x 32 rows): 16 k-steps over head_dim. kb: the
// lane's operand address in the tile's slot before the per-step XOR.
__device__ __attribute__((always_inline)) inline float16_t scores(const Rows& rw, unsigned kb) {
  float16_t s{};
#pragma unroll
  for (unsigned st = 0; st < 16; ++st)
    s = __builtin_amdgcn_mfma_f32_32x32x16_f16(lds_read_b128(kb ^ (32u * st)), rw.q[st], s, 0, 0,
                                               0);
  return s;
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

// The scores of one tile as the softmax consumes them: S^T values of the lane (keys 8 (r / 4) +
// 4 hi + r % 4 of the tile, row col) in log2 units relative to the reference max m, with the
// causal mask applied, and the factor by which O and l were scaled when m moved for this tile.
struct Pending {
  float s[16];
  float corr;
};

// Scores of a finished S^T accumulator (relative to m) -> Pending: mask (keys past lim, diagonal
// tiles only), row max over the 32 keys (16 per lane half), and the lazy rescale decision: m
// moves only when the tile exceeds it by more than the slack, wave-uniformly. The work is split
// into part(0) .. part(4) so it can sit between MFMAs; after part(4), `moved` says whether m moved
// (by `delta` >= 0 in the lane's row), and the caller must then finish(): shift the pending
// scores, reset the accumulator init, and scale O by pend.corr before the tile's P V is added.
template <bool kMasked>
struct Decide {
  float run, delta;
  bool moved;
  __device__ __attribute__((always_inline)) inline void part(unsigned i, const float16_t& acc,
                                                              Pending& pend, Rows& rw, unsigned k0,
                                                              unsigned lim, unsigned hi) {
    if (i < 4) {  // read 4 scores, mask, running max
#pragma unroll
      for (unsigned j = 0; j < 4; ++j) {
        const unsigned r = 4 * i + j;
        float x = acc[r];
        asm volatile("" : "+v"(x));  // the pending scores live in VGPRs, not in the accumulator
        if (kMasked) {
          const unsigned key = k0 + 8 * (r / 4) + 4 * hi + (r % 4);
          x = key <= lim ? x : -__builtin_inff();
        }
        pend.s[r] = x;
      }
      const float* v = pend.s + 4 * i;
      run = i == 0 ? max3(v[0], v[1], v[2]) : max3(run, v[0], v[1]);
      run = i == 0 ? max3(run, v[3], v[3]) : max3(run, v[2], v[3]);
    } else if (i == 4) {
      const float mx = cdna4::max_xor32(run);
      moved = __builtin_amdgcn_ballot_w64(mx > kRescaleSlack) != 0;
      delta = moved ? fmaxf(mx, 0.0f) : 0.0f;
      pend.corr = __builtin_amdgcn_exp2f(-delta);
      rw.m += delta;
    }
  }
  __device__ __attribute__((always_inline)) inline void finish(Pending& pend, Rows& rw) {
#pragma unroll
    for (int r = 0; r < 16; ++r)
      pend.s[r] -= delta;
    rw.negm = splat16(-rw.m);
    asm volatile("" : "+a"(rw.negm));  // kept where the MFMA reads its accumulator input
  }
};

// The first tile of an item: O and l are still 0, so m is simply the tile's row max.
template <bool kMasked>
__device__ __attribute__((always_inline)) inline void first_tile(const float16_t& acc,
                                                                Pending& pend, Rows& rw,
                                                                unsigned lim, unsigned hi) {
  float x[16];
#pragma unroll
  for (unsigned r = 0; r < 16; ++r) {
    x[r] = acc[r];
    if (kMasked) {
      const unsigned key = 8 * (r / 4) + 4 * hi + (r % 4);
      x[r] = key <= lim ? x[r] : -__builtin_inff();
    }
  }
  float run = max3(x[0], x[1], x[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2)
    run = max3(run, x[r], x[r + 1]);
  rw.m = cdna4::max_xor32(fmaxf(run, x[15]));  // finite: key 0 is visible to every row
#pragma unroll
  for (int r = 0; r < 16; ++r)
    pend.s[r] = x[r] - rw.m;
  pend.corr = 0.0f;
  rw.negm = splat16(-rw.m);
  asm volatile("" : "+a"(rw.negm));
}

// One tile of a wave, software-pipelined: tile ti's softmax numerators (from `cur`, decided in
// the previous step), O += V^T(ti) P^T(ti), and the scores of tile ti + 1 (kNext), which are
// decided at the end into `cur` for the next step. Three groups of MFMAs, each with the VALU work
// that depends only on earlier groups, interleaved one MFMA at a time (scheduling barriers):
//   A: S(ti + 1) k-steps 0-7; numerators of keys r = 0-7 -> P half 0, their sum;
//   B: S(ti + 1) k-steps 8-15 alternating with the P V MFMAs of key step 0; numerators r = 8-15;
//   C: the P V MFMAs of key step 1; scores of tile ti + 1 read, masked (kMaskNext) and decided.
// If m moved for tile ti + 1, O (now holding every tile <= ti) is rescaled at the end.
// k-slot 8 hi + j of a P V step holds key 16 step + 4 hi + (j < 4 ? j : j + 4), which is how the
// S^T accumulator rows lie in the lane, so P^T is the numerators as they are. kb: K operand
// address in slot 0 and
// k_off the byte offset of tile ti + 1's slot; vb[c] + v_off: the V^T transpose-read address of
// 32-dim block c (rows 0-7 of key step 0) in tile ti's slot. Block b + 4 lies 256 bytes above
// block b and rows 8-15 4096 +- 256 bytes above rows 0-7, so four lane bases serve all 32 reads
// (the rest are instruction offsets).
template <bool kMaskNext, bool kNext>
__device__ __attribute__((always_inline)) inline void tile_step(Pending& cur, Rows& rw,
                                                               float16_t (&o)[8], unsigned kb,
                                                               unsigned k_off,
                                                               const unsigned (&vb)[4],
                                                               unsigned v_off, unsigned k0_next,
                                                               unsigned lim, unsigned hi) {
  const unsigned ks = kb + k_off;  // k_off has no bits below 14: the XORs below commute with it
  unsigned vt[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    vt[c] = opaque(vb[c] + v_off);
  half8_t ka[16];
  float16_t s_acc;
  auto kread = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext && st < 16)
      ka[st] = lds_read_b128(ks ^ (32u * st));
  };
  auto smma = [&](unsigned st) __attribute__((always_inline)) {
    if (kNext)
      s_acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[st], rw.q[st],
                                                     st == 0 ? rw.negm : s_acc, 0, 0, 0);
  };
  // V^T operands in MFMA order (key step 0 for blocks 0-7, then key step 1), four ahead.
  constexpr unsigned kAhead = 4;
  half4_t vlo[kAhead], vup[kAhead];
  auto vread = [&](unsigned i) __attribute__((always_inline)) {
    if (i < 16) {
      const unsigned b = i % 8, step = i / 8;
      const unsigned at = vt[b % 4] + 256u * (b / 4) + 8192u * step;
      vlo[i % kAhead] = read_tr(at);
      vup[i % kAhead] = read_tr(at + (b < 4 ? 4096u + 256u : 4096u - 256u));
    }
  };
  half8_t p[2];
  auto pv = [&](unsigned i) __attribute__((always_inline)) {
    const half4_t lo = vlo[i % kAhead], up = vup[i % kAhead];
    const half8_t av = half8_t{lo[0], lo[1], lo[2], lo[3], up[0], up[1], up[2], up[3]};
    vread(i + kAhead);
    o[i % 8] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, p[i / 8], o[i % 8], 0, 0, 0);
  };
  // Numerators e(r) = 2^s(r) (s is relative to m) as f16 pairs, one exponential per call
  // (num(2 j) and num(2 j + 1) make pair j: keys r = 2 j, 2 j + 1); their sum, of the rounded
  // values the MFMAs use, by dot products with (1, 1).
  const cdna4::half2_t ones{static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
  cdna4::half2_t e2[8];
  float x_even[8];
  float lsum = 0.0f;
  auto num = [&](unsigned r) __attribute__((always_inline)) {
    const float x = __builtin_amdgcn_exp2f(cur.s[r]);
    if (r % 2 == 0) {
      x_even[r / 2] = x;
    } else {
      e2[r / 2] = cdna4::half2_t{static_cast<_Float16>(x_even[r / 2]), static_cast<_Float16>(x)};
      lsum = __builtin_amdgcn_fdot2(e2[r / 2], ones, lsum, false);
    }
  };
  auto pack = [&](unsigned h) __attribute__((always_inline)) {
    p[h] = half8_t{e2[4 * h][0],     e2[4 * h][1],     e2[4 * h + 1][0], e2[4 * h + 1][1],
                   e2[4 * h + 2][0], e2[4 * h + 2][1], e2[4 * h + 3][0], e2[4 * h + 3][1]};
  };

  // Group A.
  kread(0);
  kread(1);
#pragma unroll
  for (unsigned st = 0; st < 8; ++st) {
    kread(st + 2);
    smma(st);
    num(st);
    if (st == 3)
      vread(0), vread(1);
    if (st == 7)
      vread(2), vread(3);
    __builtin_amdgcn_sched_barrier(0);
  }
  pack(0);
  // Group B.
#pragma unroll
  for (unsigned j = 0; j < 8; ++j) {
    kread(j + 10);
    smma(j + 8);
    num(8 + j);
    pv(j);
    __builtin_amdgcn_sched_barrier(0);
  }
  pack(1);
  rw.l = rw.l * cur.corr + lsum;
  // Group C.
  Decide<kMaskNext> dec;
#pragma unroll
  for (unsigned j = 0; j < 8; ++j) {
    pv(8 + j);
    if (kNext && j >= 1 && j <= 5)
      dec.part(j - 1, s_acc, cur, rw, k0_next, lim, hi);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (kNext && dec.moved) {
    dec.finish(cur, rw);
    scale_acc(o, cur.corr);
  }
}

}  // namespace prefill_detail

// Items [first, first + count) (grid-stride). Item -> (KV head, token block) as described at
// attn_prefill_items. Per workgroup: tokens [16 b, 16 b + 16) x 8 heads of one KV head; wave w
// owns tokens 16 b + 4 w .. + 4, the 32 query rows of one MFMA column block (row n = token offset
// n / 8, head n % 8).
//
// K/V tiles of 32 keys stream into a 3-stage LDS ring by direct global->LDS loads; one barrier
// per tile. Per tile i (tile_step): the numerators of tile i, O^T += V^T P^T(i) (16 MFMAs, V^T
// from ds_read_b64_tr_b16) and S^T(i + 1) = K Q^T (16 MFMAs, Q^T resident as f16 pre-scaled by
// log2(e)/16), whose row max and rescale decision close the step. Keys past a row's causal limit
// are masked only in the diagonal tiles of a wave; the gate and 1/l are applied at the store.
template <int kBlock>
__device__ void attn_prefill_op(const AttnPrefillParams& p, unsigned first, unsigned count) {
  using namespace prefill_detail;
  using attn::kDim;
  static_assert(kBlock == 256, "four waves per prefill workgroup");
  constexpr int kGroup = attn::kQHeads / attn::kKvHeads;
  constexpr unsigned kWaveTokens = kAttnQBlock / 4;
  __shared__ Shared sh;
  const unsigned t = threadIdx.x, lane = t & 63u;
  const unsigned wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const unsigned col = lane & 31u, hi = lane >> 5;  // MFMA column / lane half
  const unsigned blocks = (p.n + kAttnQBlock - 1) / kAttnQBlock;
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
    // Ring slots as byte offsets, rotated once per tile: tile ti is in `cur`, ti + 1 in `next`,
    // ti + 2 goes to `spare`.
    unsigned slot_cur = 0, slot_next = kTileBytes, slot_spare = 2 * kTileBytes;
    auto rotate = [&]() __attribute__((always_inline)) {
      const unsigned t = slot_cur;
      slot_cur = slot_next;
      slot_next = slot_spare;
      slot_spare = t;
    };
    auto copy = [&](unsigned ti, unsigned slot) __attribute__((always_inline)) {
      const unsigned k_lds = lds0 + slot + wave * 4096;
      const unsigned v_lds = lds0 + kVBase + slot + wave * 4096;
      if ((ti + 1) * kKeys <= kv_end)
        copy_tile(K + std::size_t{ti} * kKeys * kDim, V + std::size_t{ti} * kKeys * kDim,
                  copy_koff, copy_voff, k_lds, v_lds);
      else
        copy_tile_clamped(K, V, ti * kKeys, kv_end - 1, k_lds - wave * 4096,
                          v_lds - wave * 4096, wave, lane);
    };

    // Start streaming before anything else: tiles 0 and 1.
    copy(0, slot_cur);
    if (tiles > 1)
      copy(1, slot_next);

    // This wave's rows: token tq = tw + col / 8, head kvh * 8 + col % 8.
    const unsigned tw = t0 + kWaveTokens * wave, hq = col % kGroup;
    const unsigned raw_t = tw + col / kGroup;
    const bool q_valid = raw_t < p.n;
    const unsigned tq = q_valid ? raw_t : p.n - 1;
    const unsigned lim = p.pos0 + tq;  // last visible key
    const bool wave_active = tw < p.n;
    // Tiles this wave needs, and how many of them every row of the wave sees in full (always
    // fewer: the last tile of a wave is a diagonal one).
    const unsigned wave_tiles =
        wave_active ? (p.pos0 + min(tw + kWaveTokens - 1, p.n - 1)) / kKeys + 1 : 0;
    const unsigned full_tiles = wave_active ? (p.pos0 + tw + 1) / kKeys : 0;

    Rows rw;
    {
      constexpr float kScale = kLog2e / 16.0f;  // 1/sqrt(256) in log2 units
      const float* src =
          p.q + (std::size_t{tq} * attn::kQHeads + kvh * kGroup + hq) * kDim + 8 * hi;
      const float z = q_valid ? kScale : 0.0f;
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const float4 x0 = *reinterpret_cast<const float4*>(src + 16 * st);
        const float4 x1 = *reinterpret_cast<const float4*>(src + 16 * st + 4);
        rw.q[st] = half8_t{static_cast<_Float16>(x0.x * z), static_cast<_Float16>(x0.y * z),
                           static_cast<_Float16>(x0.z * z), static_cast<_Float16>(x0.w * z),
                           static_cast<_Float16>(x1.x * z), static_cast<_Float16>(x1.y * z),
                           static_cast<_Float16>(x1.z * z), static_cast<_Float16>(x1.w * z)};
      }
      rw.m = 0.0f;
      rw.l = 0.0f;
      rw.negm = float16_t{};
    }
    float16_t oacc[8];
#pragma unroll
    for (int b = 0; b < 8; ++b)
      oacc[b] = float16_t{};

    // Start of iteration ti: tile ti + 1 complete in LDS -- this wave's share by vmcnt (it is the
    // only copy in flight), every wave's by the barrier, which also says that all waves are done
    // with tile ti - 1, whose slot then receives tile ti + 2.
    auto sync_copy = [&](unsigned ti) __attribute__((always_inline)) {
      if (ti + 1 < tiles) {
        cdna4::wait_vmcnt<0>();
        __syncthreads();
        if (ti + 2 < tiles)
          copy(ti + 2, slot_spare);
      }
    };

    cdna4::wait_vmcnt<0>();  // tiles 0 (and 1) and the queries are in
    __syncthreads();
    // cur: the decided scores of tile ti at the top of iteration ti (tile 0: here; O is still 0,
    // so the first decision needs no rescale).
    Pending cur;
    if (wave_tiles > 0) {
      const float16_t s0 = scores(rw, kb);
      if (full_tiles > 0)
        first_tile<false>(s0, cur, rw, lim, hi);
      else
        first_tile<true>(s0, cur, rw, lim, hi);
    }
    // One pass over the workgroup's tiles in phases per wave, each a loop with a single body
    // (the per-wave bounds differ; every wave still runs sync_copy once per tile, in order):
    // tiles whose successor the wave's rows see in full, tiles whose successor is diagonal, the
    // last tile (no successor), then the tiles the wave does not need.
    unsigned ti = 0;
    for (; ti + 1 < full_tiles; ++ti, rotate()) {
      sync_copy(ti);
      tile_step<false, true>(cur, rw, oacc, kb, slot_next, vb, slot_cur, (ti + 1) * kKeys, lim,
                             hi);
    }
    for (; ti + 1 < wave_tiles; ++ti, rotate()) {
      sync_copy(ti);
      tile_step<true, true>(cur, rw, oacc, kb, slot_next, vb, slot_cur, (ti + 1) * kKeys, lim, hi);
    }
    if (ti < wave_tiles) {
      sync_copy(ti);
      tile_step<false, false>(cur, rw, oacc, kb, 0, vb, slot_cur, 0, lim, hi);
      ++ti;
      rotate();
    }
    for (; ti < tiles; ++ti, rotate())
      sync_copy(ti);
    __syncthreads();  // the ring is reused by the next item

    // Row total: each column's keys per tile were split between the lane halves.
    const float l_tot = cdna4::sum_xor32(rw.l);
    if (q_valid) {
      const unsigned head = kvh * kGroup + hq;
      const float inv_l = __builtin_amdgcn_rcpf(l_tot);
      const float* gate = p.qg + std::size_t{tq} * p.qg_stride + head * 2 * kDim + kDim;
      float* out = p.core + (std::size_t{tq} * attn::kQHeads + head) * kDim;
      // Every gate load before the first store: the compiler cannot tell qg from core apart, so
      // interleaved, each load would wait behind the previous store (32 memory round trips).
      float4 gv[8][4];
#pragma unroll
      for (int b = 0; b < 8; ++b)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          gv[b][r4] = *reinterpret_cast<const float4*>(gate + 32 * b + 8 * r4 + 4 * hi);
#pragma unroll
      for (int b = 0; b < 8; ++b) {
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const unsigned d0 = 32 * b + 8 * r4 + 4 * hi;
          const float4 g = gv[b][r4];
          float4 o;
          o.x = oacc[b][4 * r4 + 0] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-g.x));
          o.y = oacc[b][4 * r4 + 1] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-g.y));
          o.z = oacc[b][4 * r4 + 2] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-g.z));
          o.w = oacc[b][4 * r4 + 3] * inv_l * __builtin_amdgcn_rcpf(1.0f + __expf(-g.w));
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
