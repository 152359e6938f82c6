// Eager timing loops for bench.py: back-to-back calls of the product's C ABI on one stream
// between two hipEvents -- the method of the reference's own bench (bench/attention/
// bench_attention.hip:24-33: hipEventRecord, n calls, hipEventRecord, hipEventElapsedTime). A
// Python caller cannot issue ~15 us calls back to back (its per-call overhead is of that order),
// so the loop runs here. Built as libmiso_bench.so next to libmiso_attn.so; nothing in the
// product loads it.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "miso_attn.h"

namespace {

struct Timer {
  hipEvent_t a = nullptr, b = nullptr;
  Timer() {
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)
      a = b = nullptr;
  }
  ~Timer() {
    if (a)
      (void)hipEventDestroy(a);
    if (b)
      (void)hipEventDestroy(b);
  }
};

}  // namespace

extern "C" {

// ms per call of `iters` calls after `warmup` untimed ones, rotating over n_buf K/V caches
// (k[i % n_buf], v[i % n_buf]). mode 0: miso_attn_decode (split + combine); 1: miso_attn_split;
// 2: miso_attn_combine (over the partials already in part_*); 3: miso_attn_decode_f16q;
// 4: miso_attn_split_valu; 5: miso_attn_decode_fused (sync: its counters).
// Returns a negative value if a call or an event fails.
double miso_bench_decode(int mode, const float* q, const float* qg, const uint16_t* const* k,
                         const uint16_t* const* v, int n_buf, float* core, float* part_m,
                         float* part_l, float* part_o, uint32_t len, uint32_t max_ctx,
                         uint32_t n_splits, int warmup, int iters, void* stream, uint32_t* sync) {
  if (n_buf < 1 || iters < 1 || warmup < 0 || mode < 0 || mode > 5 ||
      (mode == 5 && sync == nullptr))
    return -1.0;
  auto call = [&](int i) {
    const uint16_t* kc = k[i % n_buf];
    const uint16_t* vc = v[i % n_buf];
    switch (mode) {
      case 0:
        return miso_attn_decode(q, qg, kc, vc, core, part_m, part_l, part_o, len, max_ctx,
                                n_splits, stream);
      case 1:
        return miso_attn_split(q, kc, vc, part_m, part_l, part_o, len, max_ctx, n_splits, stream);
      case 2:
        return miso_attn_combine(part_m, part_l, part_o, qg, core, n_splits, stream);
      case 4:
        return miso_attn_split_valu(q, kc, vc, part_m, part_l, part_o, len, max_ctx, n_splits,
                                    stream);
      case 5:
        return miso_attn_decode_fused(q, qg, kc, vc, core, part_m, part_l, part_o, sync, len,
                                      max_ctx, n_splits, stream);
      default:
        return miso_attn_decode_f16q(q, qg, kc, vc, core, part_m, part_l, part_o, len, max_ctx,
                                     n_splits, stream);
    }
  };
  Timer t;
  if (!t.a)
    return -2.0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  for (int i = 0; i < warmup; ++i)
    if (call(i) != 0)
      return -3.0;
  if (hipEventRecord(t.a, s) != hipSuccess)
    return -2.0;
  for (int i = 0; i < iters; ++i)
    if (call(i) != 0)
      return -3.0;
  if (hipEventRecord(t.b, s) != hipSuccess || hipEventSynchronize(t.b) != hipSuccess)
    return -2.0;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess)
    return -2.0;
  return static_cast<double>(ms) / iters;
}

// ms per token of `iters` eager layer decode steps (miso_attn_layer_decode) at positions len0,
// len0 + 1, ... -- the cache grows by one row per call, as in the reference's layer bench
// (bench/attention/bench_attention.hip:22-33: 64 attention_decode calls between two events at
// each context). One untimed step at len0 first (the timed steps then overwrite its row).
// Returns a negative value if a call or an event fails.
double miso_bench_layer_decode(const miso_attn_layer* layer, uint16_t* k, uint16_t* v,
                               uint32_t len0, uint32_t max_ctx, float* h, float* y, float eps,
                               float* ws, int iters, void* stream) {
  if (iters < 1 || uint64_t{len0} + static_cast<uint32_t>(iters) > max_ctx)
    return -1.0;
  Timer t;
  if (!t.a)
    return -2.0;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (miso_attn_layer_decode(layer, k, v, len0, max_ctx, h, nullptr, y, eps, ws, stream) != 0)
    return -3.0;
  if (hipEventRecord(t.a, s) != hipSuccess)
    return -2.0;
  for (int i = 0; i < iters; ++i)
    if (miso_attn_layer_decode(layer, k, v, len0 + i, max_ctx, h, nullptr, y, eps, ws, stream) !=
        0)
      return -3.0;
  if (hipEventRecord(t.b, s) != hipSuccess || hipEventSynchronize(t.b) != hipSuccess)
    return -2.0;
  float ms = 0.0f;
  if (hipEventElapsedTime(&ms, t.a, t.b) != hipSuccess)
    return -2.0;
  return static_cast<double>(ms) / iters;
}

}  // extern "C"
