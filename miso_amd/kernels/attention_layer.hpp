#pragma once

// One gated full-attention layer step on MI355X (gfx950): the host wiring of the engine's
// attention_decode / attention_prefill (src/engine/attention.hip:76-148) over this repository's
// kernels, with the engine sizing retuned for one MI355X (256 CUs, 288 GB HBM3E):
//
//   constant            reference                              here   why (one MI355X)
//   max decode splits   60   (src/engine/attention.hpp:46)      128   C2 (32768 keys): 18.7 us vs
//                                                                     19.9 us per decode call on
//                                                                     one box (256 workgroups)
//   prefill chunk       512  (src/engine/model.hpp:58)          4096  an 8192-token prompt's
//                                                                     attention: 0.73 ms vs 2.17
//                                                                     ms (512 workgroups fill the
//                                                                     256 CUs; 512 tokens, 64)
//   prefill threshold   8    (src/engine/model.hpp:80)          12    at 4096 keys one prefill of
//                                                                     n tokens beats n decode
//                                                                     steps from n = 12
//
// Decode step (one token at position len): residual add + RMSNorm of h, the q / k / v projections
// of the normed row in one launch (qkv_gemv_kernel: Q4_K q and k, Q6_K v, K = 2048; any other
// format mix falls back to one GEMV per matrix), the per-head norms, RoPE and the K/V append
// (attn_prep), split-K attention over len + 1 keys with the LSE merge and the gate (attn_split +
// attn_combine), and the output projection. Prefill step (n tokens at pos0): the same with the
// prefill GEMMs (qgemm_act + qgemm) for the projections, attn_prep_batch, and the causal
// attn_prefill. ingest() applies the engine's policy to a run of n tokens: below the threshold one
// decode step per token, otherwise prefill chunks of at most the chunk size.
//
// Every routine returns nullptr on success or a message naming the rejected argument; the C ABI
// returns it as an error code, an engine front end can throw it.

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "attention_decode.hpp"
#include "attention_prefill.hpp"
#include "cdna4_wave.hpp"
#include "mixed_gemv.hpp"
#include "qgemm.hpp"

namespace miso::kernels::layer {

inline constexpr unsigned kMaxSplits = 128;
inline constexpr unsigned kMaxChunk = 4096;
inline constexpr unsigned kPrefillMinTokens = 12;

inline constexpr unsigned kHidden = 2048;  // residual width
inline constexpr unsigned kProj = 9216;    // [q + gate 8192 | k 512 | v 512]
inline constexpr unsigned kCore = 4096;    // 16 heads x 256

enum class Format : int { Q4K = 0, Q6K = 1 };

// A quantized matrix of n rows by k columns in its r1 layout.
struct Matrix {
  const std::uint8_t* data;
  Format format;
  unsigned n, k;
};

// The layer's weights (device): q (8192 x 2048: per head 256 query rows then 256 gate rows), k and
// v (512 x 2048), o (2048 x 4096); attn_norm [2048], q_norm / k_norm [256] (GGUF stores 1 + w);
// inv_freq [32].
struct Weights {
  Matrix q, k, v, o;
  const float* attn_norm;
  const float* q_norm;
  const float* k_norm;
  const float* inv_freq;
};

// ------------------------------------------------------------------------------------------------
// Residual add + RMSNorm of a 2048-wide row (src/engine/attention.hip:83-85 launches the
// reference's add_rmsnorm_kernel; this one is written for 256 threads x 8 elements): h += delta
// (delta may be null), out = h / sqrt(mean(h^2) + eps) * weight.
// ------------------------------------------------------------------------------------------------

struct AddRmsNormParams {
  float* h;            // [tokens][2048], updated in place when delta is set
  const float* delta;  // [tokens][2048] or nullptr
  const float* weight;  // [2048]
  float* out;           // [tokens][2048]
  float eps;
};

template <int = 0>  // a template: header-defined kernels must not clash across translation units
__global__ void __launch_bounds__(256) add_rmsnorm_kernel(AddRmsNormParams p) {
  __shared__ float wave_ss[4];
  const std::size_t row = std::size_t{blockIdx.x} * kHidden;
  const unsigned e = 8 * threadIdx.x;
  float v[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float4 a = *reinterpret_cast<const float4*>(p.h + row + e + 4 * i);
    if (p.delta != nullptr) {
      const float4 d = *reinterpret_cast<const float4*>(p.delta + row + e + 4 * i);
      a = float4{a.x + d.x, a.y + d.y, a.z + d.z, a.w + d.w};
      *reinterpret_cast<float4*>(p.h + row + e + 4 * i) = a;
    }
    v[4 * i] = a.x, v[4 * i + 1] = a.y, v[4 * i + 2] = a.z, v[4 * i + 3] = a.w;
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    ss = __builtin_fmaf(v[i], v[i], ss);
  ss = cdna4::wave_allsum(ss);
  if (threadIdx.x % 64 == 0)
    wave_ss[threadIdx.x / 64] = ss;
  __syncthreads();
  const float total = (wave_ss[0] + wave_ss[1]) + (wave_ss[2] + wave_ss[3]);
  const float r = 1.0f / __builtin_sqrtf(total * (1.0f / kHidden) + p.eps);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float4 w = *reinterpret_cast<const float4*>(p.weight + e + 4 * i);
    *reinterpret_cast<float4*>(p.out + row + e + 4 * i) =
        float4{v[4 * i] * r * w.x, v[4 * i + 1] * r * w.y, v[4 * i + 2] * r * w.z,
               v[4 * i + 3] * r * w.w};
  }
}

// ------------------------------------------------------------------------------------------------
// Projections
// ------------------------------------------------------------------------------------------------

// Decode GEMV launch shapes, from a sweep at the engine's projections (f16 activations,
// HBM-resident weights, graph-replayed): up to 1024 rows, workgroups of max(128, K / 32) threads
// with one pass per wave; more rows, 4-wave workgroups with two passes (one for K = 8192).
template <ActFormat A, unsigned K, int kBlock, int kRows>
inline void launch_q4k_gemv(const Q4kGemvParams& p, hipStream_t stream) {
  const unsigned per_wg = (kBlock / 64) * q4k_gemv_wave_rows<K, kRows>();
  unsigned grid = (p.n_rows + per_wg - 1) / per_wg;
  grid = grid < 8192u ? grid : 8192u;  // grid-stride beyond
  q4k_gemv_kernel<A, K, kBlock, kRows><<<grid, kBlock, 0, stream>>>(p);
}

template <ActFormat A, unsigned K>
inline void q4k_gemv(const Q4kGemvParams& p, hipStream_t stream) {
  if (p.n_rows <= 1024)
    launch_q4k_gemv<A, K, (K / 32 > 128 ? K / 32 : 128), 1>(p, stream);
  else
    launch_q4k_gemv<A, K, 256, (K == 8192 ? 1 : 2)>(p, stream);
}

template <unsigned K, int kBlock, int kRows>
inline void launch_q6k_gemv(const Q6kGemvParams& p, hipStream_t stream) {
  const unsigned per_wg = (kBlock / 64) * q6k_gemv_wave_rows<K, kRows>();
  unsigned grid = (p.n_rows + per_wg - 1) / per_wg;
  grid = grid < 8192u ? grid : 8192u;
  q6k_gemv_kernel<K, kBlock, kRows><<<grid, kBlock, 0, stream>>>(p);
}

template <unsigned K>
inline void q6k_gemv(const Q6kGemvParams& p, hipStream_t stream) {
  if (p.n_rows <= 1024)
    launch_q6k_gemv<K, (K / 32 > 128 ? K / 32 : 128), 1>(p, stream);
  else
    launch_q6k_gemv<K, 256, (K == 8192 ? 1 : 2)>(p, stream);
}

// y = W x for one token (f16 activations, the engine's choice).
inline const char* gemv(const Matrix& w, const float* x, float* y, hipStream_t stream) {
  if (w.n == 0)
    return nullptr;
  if (w.k != 2048 && w.k != 4096 && w.k != 8192)
    return "GEMV k must be 2048, 4096 or 8192";
  if (w.format == Format::Q4K) {
    const Q4kGemvParams p{w.data, x, y, w.n};
    if (w.k == 2048) q4k_gemv<ActFormat::Fp16, 2048>(p, stream);
    else if (w.k == 4096) q4k_gemv<ActFormat::Fp16, 4096>(p, stream);
    else q4k_gemv<ActFormat::Fp16, 8192>(p, stream);
  } else if (w.format == Format::Q6K) {
    const Q6kGemvParams p{w.data, x, y, w.n};
    if (w.k == 2048) q6k_gemv<2048>(p, stream);
    else if (w.k == 4096) q6k_gemv<4096>(p, stream);
    else q6k_gemv<8192>(p, stream);
  } else {
    return "weight format must be Q4_K (0) or Q6_K (1)";
  }
  return nullptr;
}

// The q / k / v projections of xn into proj = [q + gate | k | v]: the model's mix (Q4_K q and k,
// Q6_K v) in one launch, anything else one GEMV per matrix.
inline void qkv_launch(const Weights& w, const float* xn, float* proj, hipStream_t stream) {
  // Logical grids sized for 8192, 512 and 512 rows (16 rows per Q4_K workgroup, 8 per Q6_K).
  constexpr unsigned kQ = 512, kK = 32, kV = 64;
  const Q4kGemvParams pq{w.q.data, xn, proj, w.q.n}, pk{w.k.data, xn, proj + 8192, w.k.n};
  const Q6kGemvParams pv{w.v.data, xn, proj + 8704, w.v.n};
  qkv_gemv_kernel<kQ, kK, kV, 256><<<kQ + kK + kV, 256, 0, stream>>>(pq, pk, pv);
}

inline const char* project_qkv(const Weights& w, const float* xn, float* proj,
                               hipStream_t stream) {
  if (w.q.format == Format::Q4K && w.k.format == Format::Q4K && w.v.format == Format::Q6K) {
    qkv_launch(w, xn, proj, stream);
    return nullptr;
  }
  if (const char* err = gemv(w.q, xn, proj, stream))
    return err;
  if (const char* err = gemv(w.k, xn, proj + 8192, stream))
    return err;
  return gemv(w.v, xn, proj + 8704, stream);
}

// The prefill GEMMs: xh / xs prepared once per input (gemm_input), then Y = W x per matrix.
inline void gemm_input(const float* x, unsigned k, unsigned n_tok, _Float16* xh, float* xs,
                       hipStream_t stream) {
  const QGemmActParams p{x, xh, xs, k, n_tok};
  const unsigned quarters = n_tok * (k / 8);  // one thread per 8 elements
  qgemm_act_kernel<<<(quarters + 255) / 256, 256, 0, stream>>>(p);
}

inline const char* gemm(const Matrix& w, const _Float16* xh, const float* xs, unsigned n_tok,
                        float* y, unsigned ldy, hipStream_t stream) {
  if (w.n == 0 || n_tok == 0)
    return nullptr;
  if (w.k % 256 != 0)
    return "GEMM k must be a multiple of 256";
  const QGemmParams p{w.data, xh, xs, y, w.k, w.n, n_tok, ldy};
  const unsigned grid = qgemm_tiles(w.n, n_tok);
  if (w.format == Format::Q4K) {
    if (const unsigned big = qgemm_big_tiles(w.n, n_tok))
      qgemm_q4k_big_kernel<><<<big, 256, 0, stream>>>(p);
    else
      qgemm_kernel<QFormat::Q4K><<<grid, 256, 0, stream>>>(p);
  } else if (w.format == Format::Q6K)
    qgemm_kernel<QFormat::Q6K><<<grid, 256, 0, stream>>>(p);
  else
    return "weight format must be Q4_K (0) or Q6_K (1)";
  return nullptr;
}

// ------------------------------------------------------------------------------------------------
// Workspaces (caller-allocated device floats; the engine's AttentionScratch and
// AttentionPrefillScratch, src/engine/attention.hpp:44-69)
// ------------------------------------------------------------------------------------------------

struct DecodeWorkspace {
  float* xn;      // [2048]
  float* proj;    // [9216]
  float* q;       // [16][256]
  float* core;    // [16][256]
  float* part_m;  // [2][kMaxSplits][8]
  float* part_l;
  float* part_o;  // [2][kMaxSplits][8][256]
};

inline constexpr std::size_t decode_workspace_floats() {
  return std::size_t{kHidden} + kProj + 2 * kCore + 2 * (2 * kMaxSplits * 8) +
         std::size_t{2} * kMaxSplits * 8 * 256;
}

// Float offset of core in a decode workspace (after part_o, xn, proj and q).
inline constexpr std::size_t decode_core_offset() {
  return std::size_t{2} * kMaxSplits * 8 * 256 + kHidden + kProj + kCore;
}

// Carves ws (16-byte aligned, decode_workspace_floats() floats); every piece stays 16-byte aligned.
inline DecodeWorkspace decode_workspace(float* ws) {
  DecodeWorkspace d;
  d.part_o = ws;
  d.xn = d.part_o + std::size_t{2} * kMaxSplits * 8 * 256;
  d.proj = d.xn + kHidden;
  d.q = d.proj + kProj;
  d.core = ws + decode_core_offset();
  d.part_m = d.core + kCore;
  d.part_l = d.part_m + 2 * kMaxSplits * 8;
  return d;
}

// The prefill workspace ends with the balanced prefill's workspace for chunks of up to
// min(max_tok, 4096) tokens (attention_prefill.hpp): its pair counters must be zero before the
// first chunk, so the whole prefill workspace is zero-filled once when it is allocated (every
// chunk leaves the counters zero).
struct PrefillWorkspace {
  float* xn;     // [max_tok][2048]
  float* proj;   // [max_tok][9216]
  float* q;      // [max_tok][16][256]
  float* core;   // [max_tok][16][256]
  float* xs;     // [max_tok][4096 / 32] GEMM input sums
  _Float16* xh;  // [max_tok][4096] GEMM input values
  char* balance;  // attn_prefill_split_workspace_bytes(min(max_tok, 4096)) bytes
};

inline constexpr std::size_t prefill_balance_floats(unsigned max_tok) {
  return (attn_prefill_split_workspace_bytes(max_tok < 4096 ? max_tok : 4096) + 15) / 16 * 4;
}

inline constexpr std::size_t prefill_workspace_floats(unsigned max_tok) {
  return std::size_t{max_tok} * (kHidden + kProj + 2 * kCore + kCore / 32 + kCore / 2) +
         prefill_balance_floats(max_tok);
}

// Float offset of core in a prefill workspace (after xn, proj and q).
inline constexpr std::size_t prefill_core_offset(unsigned max_tok) {
  return std::size_t{max_tok} * (kHidden + kProj + kCore);
}

inline PrefillWorkspace prefill_workspace(float* ws, unsigned max_tok) {
  PrefillWorkspace w;
  w.xn = ws;
  w.proj = w.xn + std::size_t{max_tok} * kHidden;
  w.q = w.proj + std::size_t{max_tok} * kProj;
  w.core = ws + prefill_core_offset(max_tok);
  w.xs = w.core + std::size_t{max_tok} * kCore;
  w.xh = reinterpret_cast<_Float16*>(w.xs + std::size_t{max_tok} * (kCore / 32));
  w.balance = reinterpret_cast<char*>(w.xh + std::size_t{max_tok} * kCore);
  return w;
}

// ------------------------------------------------------------------------------------------------
// Steps
// ------------------------------------------------------------------------------------------------

// The shapes every step assumes: the projection buffer layout and the attention's head sizes.
inline const char* check_weights(const Weights& w) {
  if (w.q.n != 8192 || w.k.n != 512 || w.v.n != 512 || w.q.k != kHidden || w.k.k != kHidden ||
      w.v.k != kHidden)
    return "q / k / v must be 8192 / 512 / 512 rows of 2048";
  if (w.o.n != kHidden || w.o.k != kCore)
    return "o must be 2048 rows of 4096";
  return nullptr;
}

// The token at position len: h += delta, y = Attention(RMSNorm(h)); K/V appended at len.
inline const char* decode_step(const Weights& w, attn::half_t* k_cache, attn::half_t* v_cache,
                               unsigned len, unsigned max_ctx, float* h, const float* delta,
                               float* y, float eps, const DecodeWorkspace& ws,
                               hipStream_t stream) {
  if (len >= max_ctx)
    return "KV cache is full";
  add_rmsnorm_kernel<<<1, 256, 0, stream>>>(AddRmsNormParams{h, delta, w.attn_norm, ws.xn, eps});
  if (const char* err = project_qkv(w, ws.xn, ws.proj, stream))
    return err;
  const AttnPrepParams prep{ws.proj,  ws.proj + 8192, ws.proj + 8704, w.q_norm, w.k_norm,
                            w.inv_freq, k_cache,      v_cache,        ws.q,     len,
                            max_ctx,  eps};
  attn_prep_kernel<256><<<18, 256, 0, stream>>>(prep);
  const unsigned keys = len + 1, n_splits = attn_n_splits(keys, kMaxSplits);
  const AttnSplitParams split{ws.q,      k_cache,   v_cache, ws.part_m, ws.part_l,
                              ws.part_o, keys,      max_ctx, n_splits};
  attn_split_kernel<256><<<dim3(n_splits, 2), 256, 0, stream>>>(split);
  const AttnCombineParams comb{ws.part_m, ws.part_l, ws.part_o, ws.proj, ws.core, n_splits};
  attn_combine_kernel<64, true, 4><<<64, 64, 0, stream>>>(comb);
  return gemv(w.o, ws.core, y, stream);
}

// n consecutive tokens at pos0 ([n][2048] h / delta / y): the prefill GEMMs, batched prep and
// causal flash attention over the cache up to each token (the balanced form for chunks of up to
// 4096 tokens).
inline const char* prefill_step(const Weights& w, attn::half_t* k_cache, attn::half_t* v_cache,
                                unsigned pos0, unsigned n, unsigned max_ctx, float* h,
                                const float* delta, float* y, float eps,
                                const PrefillWorkspace& ws, unsigned max_tok,
                                hipStream_t stream) {
  if (n == 0)
    return nullptr;
  if (n > max_tok)
    return "chunk does not fit the prefill workspace";
  if (std::size_t{pos0} + n > max_ctx)
    return "KV cache is full";
  add_rmsnorm_kernel<<<n, 256, 0, stream>>>(AddRmsNormParams{h, delta, w.attn_norm, ws.xn, eps});
  gemm_input(ws.xn, kHidden, n, ws.xh, ws.xs, stream);
  const char* err = gemm(w.q, ws.xh, ws.xs, n, ws.proj, kProj, stream);
  if (err == nullptr)
    err = gemm(w.k, ws.xh, ws.xs, n, ws.proj + 8192, kProj, stream);
  if (err == nullptr)
    err = gemm(w.v, ws.xh, ws.xs, n, ws.proj + 8704, kProj, stream);
  if (err != nullptr)
    return err;
  const AttnPrepBatchParams prep{{ws.proj, ws.proj + 8192, ws.proj + 8704, w.q_norm, w.k_norm,
                                  w.inv_freq, k_cache, v_cache, ws.q, pos0, max_ctx, eps},
                                 n,
                                 kProj};
  attn_prep_batch_kernel<256><<<n * 18, 256, 0, stream>>>(prep);
  const AttnPrefillParams ap{ws.q, ws.proj, k_cache, v_cache, ws.core, pos0, n, max_ctx, kProj};
  if (attn_prefill_balanced(n)) {  // n <= 4096 and n <= max_tok: within its workspace
    float* const part_ml = reinterpret_cast<float*>(ws.balance + kAttnSplitCounterBytes);
    const std::size_t ml_floats =
        std::size_t{attn_prefill_split_pairs(n)} * 2 * attn_prefill_split_rows(n) * 2;
    const AttnPrefillSplitParams sp{ap, part_ml + ml_floats, part_ml,
                                    reinterpret_cast<unsigned*>(ws.balance)};
    attn_prefill_split_kernel<256><<<attn_prefill_split_items(n), 256, 0, stream>>>(sp);
  } else {
    attn_prefill_kernel<256><<<attn_prefill_items(n), 256, 0, stream>>>(ap);
  }
  gemm_input(ws.core, kCore, n, ws.xh, ws.xs, stream);
  return gemm(w.o, ws.xh, ws.xs, n, y, kHidden, stream);
}

// n tokens at pos0 through the layer, the engine's policy (src/engine/model.hip:130-175 for this
// layer): fewer than kPrefillMinTokens, one decode step each; otherwise prefill chunks of at most
// `chunk` tokens (0: kMaxChunk; at most max_tok).
inline const char* ingest(const Weights& w, attn::half_t* k_cache, attn::half_t* v_cache,
                          unsigned pos0, unsigned n, unsigned max_ctx, float* h,
                          const float* delta, float* y, float eps, const DecodeWorkspace& dws,
                          const PrefillWorkspace& pws, unsigned max_tok, unsigned chunk,
                          hipStream_t stream) {
  if (std::size_t{pos0} + n > max_ctx)
    return "KV cache is full";
  if (n < kPrefillMinTokens) {
    for (unsigned t = 0; t < n; ++t) {
      const std::size_t at = std::size_t{t} * kHidden;
      if (const char* err = decode_step(w, k_cache, v_cache, pos0 + t, max_ctx, h + at,
                                        delta != nullptr ? delta + at : nullptr, y + at, eps,
                                        dws, stream))
        return err;
    }
    return nullptr;
  }
  chunk = chunk == 0 ? kMaxChunk : chunk;
  chunk = chunk < max_tok ? chunk : max_tok;
  if (chunk == 0)
    return "the prefill workspace holds no tokens";
  for (unsigned t = 0; t < n; t += chunk) {
    const unsigned m = n - t < chunk ? n - t : chunk;
    const std::size_t at = std::size_t{t} * kHidden;
    if (const char* err = prefill_step(w, k_cache, v_cache, pos0 + t, m, max_ctx, h + at,
                                       delta != nullptr ? delta + at : nullptr, y + at, eps, pws,
                                       max_tok, stream))
      return err;
  }
  return nullptr;
}

}  // namespace miso::kernels::layer
