// Source-level drop-in for the engine's src/engine/attention.hip (see attention.hpp beside it):
// the engine's types mapped onto the layer wiring of miso_amd/kernels/attention_layer.hpp.

#include "engine/attention.hpp"

#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "attention_layer.hpp"

namespace miso {
namespace {

namespace L = kernels::layer;

L::Matrix view(const QMatrix& m, const char* what) {
  if (m.type == gguf::GgmlType::Q4_K)
    return {m.data.data(), L::Format::Q4K, m.n, m.k};
  if (m.type == gguf::GgmlType::Q6_K)
    return {m.data.data(), L::Format::Q6K, m.n, m.k};
  throw std::runtime_error(std::string("attention: ") + what + " must be Q4_K or Q6_K");
}

L::Weights weights(const AttentionLayer& w, const RopeConfig& rope) {
  L::Weights out{view(w.q, "attn_q"),   view(w.k, "attn_k"),   view(w.v, "attn_v"),
                 view(w.o, "attn_output"), w.attn_norm.data(),  w.q_norm.data(),
                 w.k_norm.data(),        rope.inv_freq.data()};
  if (const char* err = L::check_weights(out))
    throw std::runtime_error(std::string("attention: ") + err);
  return out;
}

void check(const char* fn, const char* err) {
  if (err != nullptr)
    throw std::runtime_error(std::string(fn) + ": " + err);
  MISO_HIP_CHECK(hipGetLastError());
}

}  // namespace

AttentionLayer AttentionLayer::load(const gguf::File& f, int layer, LoadStage* st) {
  const std::string p = "blk." + std::to_string(layer) + ".";
  return {upload_qmatrix(f, p + "attn_q.weight", st),
          upload_qmatrix(f, p + "attn_k.weight", st),
          upload_qmatrix(f, p + "attn_v.weight", st),
          upload_qmatrix(f, p + "attn_output.weight", st),
          upload_f32(f, p + "attn_norm.weight", st),
          upload_f32(f, p + "attn_q_norm.weight", st),
          upload_f32(f, p + "attn_k_norm.weight", st)};
}

RopeConfig RopeConfig::from(const gguf::File& f) {
  const double base = f.get<double>("qwen35moe.rope.freq_base");
  const auto dims = f.get<std::int64_t>("qwen35moe.rope.dimension_count");
  constexpr int kRot = kernels::attn::kRopeDim;
  if (dims != kRot)
    throw std::runtime_error("attention: the kernels rotate 64 dimensions per head");
  // inv_freq[i] = 1 / base^(2 i / 64), evaluated in f32 as transformers does.
  std::vector<float> inv(kRot / 2);
  for (int i = 0; i < kRot / 2; ++i)
    inv[i] = 1.0f / std::pow(static_cast<float>(base), static_cast<float>(2 * i) / kRot);
  return {DeviceBuffer<float>(inv)};
}

AttentionCache::AttentionCache(unsigned n)
    : max_ctx(n), k(std::size_t{2} * n * 256), v(std::size_t{2} * n * 256) {}

AttentionPrefillScratch::AttentionPrefillScratch(unsigned n)
    : max_tok(n),
      in(n, L::kCore),
      xn(std::size_t{n} * L::kHidden),
      proj(std::size_t{n} * AttentionScratch::kProj),
      q(std::size_t{n} * L::kCore),
      core(std::size_t{n} * L::kCore),
      balance(L::prefill_balance_floats(n)) {
  // The balanced prefill's pair counters start at zero (every chunk leaves them so).
  if (balance.size() != 0)
    MISO_HIP_CHECK(hipMemset(balance.data(), 0, balance.size() * sizeof(float)));
}

void attention_decode(const AttentionLayer& w, AttentionCache& cache, AttentionScratch& sc,
                      const RopeConfig& rope, float* h, const float* delta, float* y, float eps,
                      hipStream_t stream) {
  static_assert(AttentionScratch::kMaxSplits == L::kMaxSplits, "one split cap");
  static_assert(AttentionScratch::kProj == L::kProj, "one projection layout");
  auto* kc = reinterpret_cast<kernels::attn::half_t*>(cache.k.data());
  auto* vc = reinterpret_cast<kernels::attn::half_t*>(cache.v.data());
  const L::DecodeWorkspace ws{sc.xn.data(),     sc.proj.data(),   sc.q.data(),     sc.core.data(),
                              sc.part_m.data(), sc.part_l.data(), sc.part_o.data()};
  check("attention_decode", L::decode_step(weights(w, rope), kc, vc, cache.len, cache.max_ctx, h,
                                           delta, y, eps, ws, stream));
  ++cache.len;
}

void attention_prefill(const AttentionLayer& w, AttentionCache& cache, AttentionScratch& sc,
                       AttentionPrefillScratch& ps, const RopeConfig& rope, float* h,
                       const float* delta, float* y, unsigned n, float eps, hipStream_t stream) {
  (void)sc;  // the prefill wiring has its own workspace
  auto* kc = reinterpret_cast<kernels::attn::half_t*>(cache.k.data());
  auto* vc = reinterpret_cast<kernels::attn::half_t*>(cache.v.data());
  const L::PrefillWorkspace ws{ps.xn.data(),   ps.proj.data(), ps.q.data(),
                               ps.core.data(), ps.in.xs.data(), ps.in.xh.data(),
                               reinterpret_cast<char*>(ps.balance.data())};
  check("attention_prefill", L::prefill_step(weights(w, rope), kc, vc, cache.len, n,
                                             cache.max_ctx, h, delta, y, eps, ws, ps.max_tok,
                                             stream));
  if (n != 0)  // the last GEMM input prepared: the chunk's core rows
    ps.in.k = L::kCore, ps.in.n_tok = n;
  cache.len += n;
}

}  // namespace miso
