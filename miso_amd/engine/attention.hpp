#pragma once

// Source-level drop-in for the engine's src/engine/attention.hpp: the gated full-attention token
// mixer of one layer, with the host wiring of miso_amd/kernels/attention_layer.hpp behind the
// engine's own declarations (the names, signatures and constructors src/engine/model.hpp and
// model.hip use: AttentionLayer::load, RopeConfig::from, AttentionCache, AttentionScratch,
// AttentionPrefillScratch, attention_decode, attention_prefill). Built inside the engine: it
// includes the engine's weights.hpp / gguf.hpp / hip_util.hpp. The layouts behind the names are
// this file's own: four separate weight matrices; the scratch members are the engine's.
//
// Sizing retuned for one MI355X: AttentionScratch::kMaxSplits = 128 (the engine: 60). The other
// two constants live in src/engine/model.hpp (kMaxChunk = 4096 and kPrefillMinTokens = 12 on
// MI355X; the engine: 512 and 8); the prefill scratch takes whatever chunk the session gives it.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "engine/weights.hpp"
#include "gguf.hpp"
#include "hip_util.hpp"

namespace miso {

// One layer's weights: attn_q (8192 rows: per head 256 query then 256 gate rows), attn_k and
// attn_v (512 rows each), attn_output (2048 rows of 4096), Q4_K or Q6_K each; the norms.
struct AttentionLayer {
  QMatrix q, k, v, o;
  DeviceBuffer<float> attn_norm, q_norm, k_norm;

  static AttentionLayer load(const gguf::File& f, int layer, LoadStage* st = nullptr);
};

// RoPE inverse frequencies of the rotated dimensions (f32, as transformers computes them).
struct RopeConfig {
  DeviceBuffer<float> inv_freq;

  static RopeConfig from(const gguf::File& f);
};

// f16 KV cache of one layer: [2 KV heads][max_ctx][256] for K and for V.
struct AttentionCache {
  explicit AttentionCache(unsigned max_ctx);
  unsigned max_ctx;
  unsigned len = 0;
  DeviceBuffer<std::uint16_t> k, v;
};

// Decode workspace. The members are the engine's (callers read them: the layer's output before
// the output projection is `core`, 16 heads x 256): the normed row, the [q + gate | k | v]
// projections, the prepared q, core, and the split partials for up to kMaxSplits splits.
struct AttentionScratch {
  static constexpr unsigned kMaxSplits = 128;
  static constexpr unsigned kProj = 9216;
  DeviceBuffer<float> xn{2048}, proj{kProj}, q{4096}, core{4096};
  DeviceBuffer<float> part_m{2 * kMaxSplits * 8}, part_l{2 * kMaxSplits * 8};
  DeviceBuffer<float> part_o{2 * kMaxSplits * 8 * 256};
  float* qg() { return proj.data(); }
  float* k() { return proj.data() + 8192; }
  float* v() { return proj.data() + 8704; }
};

// Prefill workspace for chunks of up to max_tok tokens, with the engine's members (`core` holds
// the last chunk's [n][16][256] attention output) plus `balance`: the balanced prefill's
// partials and pair counters for chunks of up to min(max_tok, 4096) tokens, zero-filled once here
// (every chunk leaves the counters zero).
struct AttentionPrefillScratch {
  explicit AttentionPrefillScratch(unsigned max_tok);
  unsigned max_tok;
  GemmInput in;
  DeviceBuffer<float> xn, proj, q, core;
  DeviceBuffer<float> balance;
  float* qg() { return proj.data(); }
  float* k() { return proj.data() + 8192; }
  float* v() { return proj.data() + 8704; }
};

// h += delta (when delta is set), then y = Attention(RMSNorm(h)) for the token at position
// cache.len, which is appended to the cache.
void attention_decode(const AttentionLayer& w, AttentionCache& cache, AttentionScratch& sc,
                      const RopeConfig& rope, float* h, const float* delta, float* y, float eps,
                      hipStream_t stream);

// The same for n consecutive tokens ([n][2048] arrays): prefill GEMMs, then causal attention over
// the chunk (each token sees the cache up to itself).
void attention_prefill(const AttentionLayer& w, AttentionCache& cache, AttentionScratch& sc,
                       AttentionPrefillScratch& ps, const RopeConfig& rope, float* h,
                       const float* delta, float* y, unsigned n, float eps, hipStream_t stream);

}  // namespace miso
