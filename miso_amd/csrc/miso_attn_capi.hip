// C ABI of the MI355X attention library: argument validation on the host, then launches of the
// kernels the header API defines (miso_amd/kernels/*.hpp), with the reference callers' launch
// shapes. Declarations and contracts: include/miso_attn.h.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/miso_attn.h"
#include "attention_decode.hpp"
#include "attention_decode_fp8.hpp"
#include "attention_prefill.hpp"
#include "q4k_gemv.hpp"
#include "q6k_gemv.hpp"
#include "attention_layer.hpp"
#include "mixed_gemv.hpp"
#include "qgemm.hpp"

namespace k = miso::kernels;
using k::attn::half_t;

namespace {

thread_local std::string g_last_error;

int fail(const char* fn, const char* msg) {
  g_last_error = std::string(fn) + ": " + msg;
  return MISO_ATTN_EINVAL;
}

// The reference checks hipGetLastError() after its launches (MISO_HIP_CHECK) and throws with the
// error's name; here the same error becomes the return code and the message.
int launched(const char* fn) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess)
    return 0;
  g_last_error = std::string(fn) + ": " + hipGetErrorName(err) + " (" + hipGetErrorString(err) + ")";
  return static_cast<int>(err);
}

// The GEMV launch shapes are the layer wiring's (attention_layer.hpp: a sweep at the engine's
// projections).
using k::layer::q4k_gemv;
using k::layer::q6k_gemv;

template <bool kPrepared, int kPipeline>
__global__ void __launch_bounds__(64) combine_range_kernel(k::AttnCombineParams p, unsigned first,
                                                           unsigned count) {
  k::attn_combine_op<64, kPrepared, kPipeline>(p, first, count);
}

// Tensor pointers must be non-null and 16-byte aligned: the kernels move 16 bytes per lane.
// The per-split scalars part_m / part_l are read one float at a time and need 4-byte alignment.
bool bad_ptr(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) != 0; }
bool bad_scalars(const float* p) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 3u) != 0;
}

template <class... P>
bool any_bad(const P*... p) {
  return (bad_ptr(p) || ...);
}

constexpr const char* kBadPtr = "a tensor pointer is NULL or not 16-byte aligned";

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The split partials of miso_attn_decode_noalloc: part_o [2][128][8][256], then part_m and
// part_l [2][128][8] (2,105,344 bytes per device).
constexpr uint32_t kNoAllocMaxSplits = MISO_ATTN_NOALLOC_MAX_SPLITS;
constexpr std::size_t kNoAllocStats = std::size_t{2} * kNoAllocMaxSplits * 8;
constexpr std::size_t kNoAllocFloats = kNoAllocStats * 256 + 2 * kNoAllocStats;

}  // namespace

// Device memory of the allocation-free decode (one copy per GPU, alive until the process ends).
// Host code never uses this name as an address: each device's copy is reached through the
// pointer hipGetSymbolAddress returns for it (noalloc_scratch below).
static __device__ __align__(256) float scratch[kNoAllocFloats];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float* g_scratch_ptr[kMaxDevices] = {};

// The calling thread's current device's copy of `scratch`, looked up once per device (with that
// device current) and kept; nullptr with a message on failure.
float* noalloc_scratch(const char* fn) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(fn, "no usable current device (hipGetDevice failed or id >= 64)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      g_last_error = std::string(fn) + ": hipGetSymbolAddress(scratch) failed: " +
                     hipGetErrorName(err);
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  return g_scratch_ptr[dev];
}
const half_t* as_half(const uint16_t* p) { return reinterpret_cast<const half_t*>(p); }
half_t* as_half(uint16_t* p) { return reinterpret_cast<half_t*>(p); }

}  // namespace

extern "C" {

const char* miso_attn_last_error(void) { return g_last_error.c_str(); }

const char* miso_attn_version(void) { return "miso_attn gfx950 2"; }

uint32_t miso_attn_n_splits(uint32_t len, uint32_t max_splits) {
  return k::attn_n_splits(len, max_splits);
}

uint32_t miso_attn_prefill_items(uint32_t n) { return k::attn_prefill_items(n); }

int miso_attn_prep(const float* qg, const float* kp, const float* v, const float* q_norm,
                   const float* k_norm, const float* inv_freq, uint16_t* k_cache,
                   uint16_t* v_cache, float* q, uint32_t pos, uint32_t max_ctx, float eps,
                   void* stream) {
  if (any_bad(qg, kp, v, q_norm, k_norm, inv_freq, k_cache, v_cache, q))
    return fail("miso_attn_prep", kBadPtr);
  if (pos >= max_ctx)
    return fail("miso_attn_prep", "KV cache is full (pos >= max_ctx)");
  const k::AttnPrepParams p{qg,     kp,          v,           q_norm, k_norm, inv_freq,
                            as_half(k_cache), as_half(v_cache), q, pos, max_ctx, eps};
  k::attn_prep_kernel<256><<<18, 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prep");
}

int miso_attn_prep_batch(const float* qg, const float* kp, const float* v, const float* q_norm,
                         const float* k_norm, const float* inv_freq, uint16_t* k_cache,
                         uint16_t* v_cache, float* q, uint32_t pos0, uint32_t max_ctx, float eps,
                         uint32_t n, uint32_t proj_stride, void* stream) {
  if (n == 0)
    return 0;
  if (any_bad(qg, kp, v, q_norm, k_norm, inv_freq, k_cache, v_cache, q))
    return fail("miso_attn_prep_batch", kBadPtr);
  if (static_cast<uint64_t>(pos0) + n > max_ctx)
    return fail("miso_attn_prep_batch", "KV cache is full (pos0 + n > max_ctx)");
  if (proj_stride < 8192 + 1024)
    return fail("miso_attn_prep_batch", "proj_stride must cover [q+gate 8192 | k 512 | v 512]");
  const k::AttnPrepBatchParams p{{qg, kp, v, q_norm, k_norm, inv_freq, as_half(k_cache),
                                  as_half(v_cache), q, pos0, max_ctx, eps},
                                 n,
                                 proj_stride};
  k::attn_prep_batch_kernel<256><<<n * 18, 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prep_batch");
}

int miso_attn_split(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    float* part_m, float* part_l, float* part_o, uint32_t len, uint32_t max_ctx,
                    uint32_t n_splits, void* stream) {
  if (any_bad(q, k_cache, v_cache, part_o) || bad_scalars(part_m) || bad_scalars(part_l))
    return fail("miso_attn_split", kBadPtr);
  if (len == 0)
    return fail("miso_attn_split", "len must be >= 1");
  if (len > max_ctx)
    return fail("miso_attn_split", "len exceeds max_ctx");
  if (n_splits == 0)
    return fail("miso_attn_split", "n_splits must be >= 1");
  const k::AttnSplitParams p{q,      as_half(k_cache), as_half(v_cache), part_m, part_l,
                             part_o, len,              max_ctx,          n_splits};
  k::attn_split_kernel<256><<<dim3(n_splits, 2), 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_split");
}

int miso_attn_split_valu(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         float* part_m, float* part_l, float* part_o, uint32_t len,
                         uint32_t max_ctx, uint32_t n_splits, void* stream) {
  constexpr const char* fn = "miso_attn_split_valu";
  if (any_bad(q, k_cache, v_cache, part_o) || bad_scalars(part_m) || bad_scalars(part_l))
    return fail(fn, kBadPtr);
  if (len == 0)
    return fail(fn, "len must be >= 1");
  if (len > max_ctx)
    return fail(fn, "len exceeds max_ctx");
  if (n_splits == 0)
    return fail(fn, "n_splits must be >= 1");
  const k::AttnSplitParams p{q,      as_half(k_cache), as_half(v_cache), part_m, part_l,
                             part_o, len,              max_ctx,          n_splits};
  k::attn_split_valu_kernel<256><<<dim3(n_splits, 2), 256, 0, as_stream(stream)>>>(p);
  return launched(fn);
}

int miso_attn_combine(const float* part_m, const float* part_l, const float* part_o,
                      const float* qg, float* core, uint32_t n_splits, void* stream) {
  if (any_bad(part_o, qg, core) || bad_scalars(part_m) || bad_scalars(part_l))
    return fail("miso_attn_combine", kBadPtr);
  if (n_splits == 0)
    return fail("miso_attn_combine", "n_splits must be >= 1");
  const k::AttnCombineParams p{part_m, part_l, part_o, qg, core, n_splits};
  k::attn_combine_kernel<64, true, 4><<<64, 64, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_combine");
}

int miso_attn_combine_variant(int variant, const float* part_m, const float* part_l,
                              const float* part_o, const float* qg, float* core,
                              uint32_t n_splits, uint32_t first, uint32_t count, uint32_t grid,
                              void* stream) {
  if (any_bad(part_o, qg, core) || bad_scalars(part_m) || bad_scalars(part_l))
    return fail("miso_attn_combine_variant", kBadPtr);
  if (n_splits == 0)
    return fail("miso_attn_combine_variant", "n_splits must be >= 1");
  if (variant < 0 || variant > 3)
    return fail("miso_attn_combine_variant", "variant must be 0..3");
  constexpr uint32_t kTiles = 16 * (256 / 64);
  if (count > 0 && (variant == 0 || grid == 0 || first > kTiles || count > kTiles - first))
    return fail("miso_attn_combine_variant", "range form needs variant 1..3, grid >= 1 and "
                "first + count <= 64");
  const k::AttnCombineParams p{part_m, part_l, part_o, qg, core, n_splits};
  const hipStream_t st = as_stream(stream);
  if (count == 0) {
    switch (variant) {
      case 0: k::attn_combine_kernel<256><<<16, 256, 0, st>>>(p); break;
      case 1: k::attn_combine_kernel<64><<<64, 64, 0, st>>>(p); break;
      case 2: k::attn_combine_kernel<64, true><<<64, 64, 0, st>>>(p); break;
      default: k::attn_combine_kernel<64, true, 4><<<64, 64, 0, st>>>(p); break;
    }
  } else {
    switch (variant) {
      case 1: combine_range_kernel<false, 1><<<grid, 64, 0, st>>>(p, first, count); break;
      case 2: combine_range_kernel<true, 1><<<grid, 64, 0, st>>>(p, first, count); break;
      default: combine_range_kernel<true, 4><<<grid, 64, 0, st>>>(p, first, count); break;
    }
  }
  return launched("miso_attn_combine_variant");
}

int miso_attn_decode_f16q(const float* q, const float* qg, const uint16_t* k_cache,
                          const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                          float* part_o, uint32_t len, uint32_t max_ctx, uint32_t n_splits,
                          void* stream) {
  if (any_bad(q, qg, k_cache, v_cache, core, part_o) || bad_scalars(part_m) ||
      bad_scalars(part_l))
    return fail("miso_attn_decode_f16q", kBadPtr);
  if (len == 0)
    return fail("miso_attn_decode_f16q", "len must be >= 1");
  if (len > max_ctx)
    return fail("miso_attn_decode_f16q", "len exceeds max_ctx");
  if (n_splits == 0)
    return fail("miso_attn_decode_f16q", "n_splits must be >= 1");
  const k::AttnSplitParams p{q,      as_half(k_cache), as_half(v_cache), part_m, part_l,
                             part_o, len,              max_ctx,          n_splits};
  k::attn_split_f16q_kernel<256><<<dim3(n_splits, 2), 256, 0, as_stream(stream)>>>(p);
  const int rc = launched("miso_attn_decode_f16q");
  if (rc != 0)
    return rc;
  return miso_attn_combine(part_m, part_l, part_o, qg, core, n_splits, stream);
}

int miso_attn_decode(const float* q, const float* qg, const uint16_t* k_cache,
                     const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                     float* part_o, uint32_t len, uint32_t max_ctx, uint32_t n_splits,
                     void* stream) {
  const int rc =
      miso_attn_split(q, k_cache, v_cache, part_m, part_l, part_o, len, max_ctx, n_splits, stream);
  if (rc != 0)
    return rc;
  return miso_attn_combine(part_m, part_l, part_o, qg, core, n_splits, stream);
}

// Compute units of the current device (0 if the query fails), cached per device.
static unsigned device_cus() {
  static std::mutex mu;
  static int cache[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cache[dev] = cus;
  }
  return static_cast<unsigned>(cache[dev]);
}

int miso_attn_decode_fused(const float* q, const float* qg, const uint16_t* k_cache,
                           const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                           float* part_o, uint32_t* sync, uint32_t len, uint32_t max_ctx,
                           uint32_t n_splits, void* stream) {
  constexpr const char* fn = "miso_attn_decode_fused";
  if (any_bad(q, qg, k_cache, v_cache, core, part_o, sync) || bad_scalars(part_m) ||
      bad_scalars(part_l))
    return fail(fn, kBadPtr);
  if (len == 0)
    return fail(fn, "len must be >= 1");
  if (len > max_ctx)
    return fail(fn, "len exceeds max_ctx");
  if (n_splits == 0 || n_splits > k::kAttnTargetSplits)
    return fail(fn, "n_splits must be 1..128");
  const unsigned cus = device_cus();
  if (cus == 0)
    return fail(fn, "cannot query the device's compute units");
  // Waiting mergers hold at most 2 min(n_splits, 32) CUs (one workgroup per CU: 136 KiB of LDS);
  // with no CU left for the splits still to start, run the two-launch path.
  if (cus <= 2 * k::attn_fused_mergers(n_splits))
    return miso_attn_decode(q, qg, k_cache, v_cache, core, part_m, part_l, part_o, len, max_ctx,
                            n_splits, stream);
  const k::AttnDecodeFusedParams p{
      {q, as_half(k_cache), as_half(v_cache), part_m, part_l, part_o, len, max_ctx, n_splits},
      qg,
      core,
      sync};
  k::attn_decode_fused_kernel<256><<<dim3(n_splits, 2), 256, 0, as_stream(stream)>>>(p);
  return launched(fn);
}

int miso_attn_decode_noalloc(const float* q, const float* qg, const uint16_t* k_cache,
                             const uint16_t* v_cache, float* core, uint32_t len, uint32_t max_ctx,
                             uint32_t n_splits, void* stream) {
  constexpr const char* fn = "miso_attn_decode_noalloc";
  if (any_bad(q, qg, k_cache, v_cache, core))
    return fail(fn, kBadPtr);
  if (len == 0)
    return fail(fn, "len must be >= 1");
  if (len > max_ctx)
    return fail(fn, "len exceeds max_ctx");
  if (n_splits == 0 || n_splits > kNoAllocMaxSplits)
    return fail(fn, "n_splits must be in [1, MISO_ATTN_NOALLOC_MAX_SPLITS = 128]");
  float* const base = noalloc_scratch(fn);
  if (base == nullptr)
    return MISO_ATTN_EINVAL;
  // Every partial the combine reads is written by the split first (empty spans included), so
  // nothing is cleared between calls.
  float* const part_o = base;
  float* const part_m = base + kNoAllocStats * 256;
  float* const part_l = part_m + kNoAllocStats;
  return miso_attn_decode(q, qg, k_cache, v_cache, core, part_m, part_l, part_o, len, max_ctx,
                          n_splits, stream);
}

// The argument checks of the prefill entry points (0 if the arguments are good).
static int prefill_args(const char* fn, const float* q, const float* qg, const uint16_t* k_cache,
                        const uint16_t* v_cache, float* core, uint32_t pos0, uint32_t n,
                        uint32_t max_ctx, uint32_t qg_stride) {
  if (any_bad(q, qg, k_cache, v_cache, core))
    return fail(fn, kBadPtr);
  if (n == 0)
    return fail(fn, "n must be >= 1");
  if (static_cast<uint64_t>(pos0) + n > max_ctx)
    return fail(fn, "KV cache is full (pos0 + n > max_ctx)");
  if (qg_stride < 8192 || qg_stride % 4 != 0)
    return fail(fn, "qg_stride must be >= 8192 and a multiple of 4");
  return 0;
}

int miso_attn_prefill(const float* q, const float* qg, const uint16_t* k_cache,
                      const uint16_t* v_cache, float* core, uint32_t pos0, uint32_t n,
                      uint32_t max_ctx, uint32_t qg_stride, void* stream) {
  if (const int rc = prefill_args("miso_attn_prefill", q, qg, k_cache, v_cache, core, pos0, n,
                                  max_ctx, qg_stride))
    return rc;
  const k::AttnPrefillParams p{q,    qg, as_half(k_cache), as_half(v_cache), core, pos0,
                               n,    max_ctx, qg_stride};
  k::attn_prefill_kernel<256><<<k::attn_prefill_items(n), 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prefill");
}

uint64_t miso_attn_prefill_workspace_bytes(uint32_t n) {
  return k::attn_prefill_balanced(n) ? k::attn_prefill_split_workspace_bytes(n) : 0;
}

int miso_attn_prefill_ws(const float* q, const float* qg, const uint16_t* k_cache,
                         const uint16_t* v_cache, float* core, uint32_t pos0, uint32_t n,
                         uint32_t max_ctx, uint32_t qg_stride, void* workspace,
                         uint64_t workspace_bytes, void* stream) {
  static const char* fn = "miso_attn_prefill_ws";
  if (const int rc =
          prefill_args(fn, q, qg, k_cache, v_cache, core, pos0, n, max_ctx, qg_stride))
    return rc;
  const k::AttnPrefillParams a{q,    qg, as_half(k_cache), as_half(v_cache), core, pos0,
                               n,    max_ctx, qg_stride};
  if (!k::attn_prefill_balanced(n)) {  // the one-block-per-workgroup layout
    k::attn_prefill_kernel<256><<<k::attn_prefill_items(n), 256, 0, as_stream(stream)>>>(a);
    return launched(fn);
  }
  if (bad_ptr(workspace))
    return fail(fn, "workspace must be a non-null, 16-byte aligned device pointer");
  if (workspace_bytes < k::attn_prefill_split_workspace_bytes(n))
    return fail(fn, "workspace smaller than miso_attn_prefill_workspace_bytes(n)");
  char* const ws = static_cast<char*>(workspace);
  float* const part_ml = reinterpret_cast<float*>(ws + k::kAttnSplitCounterBytes);
  float* const part_o = part_ml + std::size_t{k::attn_prefill_split_pairs(n)} * 2 *
                                       k::attn_prefill_split_rows(n) * 2;
  const k::AttnPrefillSplitParams p{a, part_o, part_ml, reinterpret_cast<unsigned*>(ws)};
  k::attn_prefill_split_kernel<256><<<k::attn_prefill_split_items(n), 256, 0,
                                      as_stream(stream)>>>(p);
  return launched(fn);
}

uint32_t miso_attn_ragged_splits(uint32_t max_len) { return k::attn_ragged_splits(max_len); }

uint32_t miso_attn_ragged_chunk(uint32_t batch, uint32_t max_len) {
  return k::attn_ragged_chunk(batch, max_len, device_cus());
}

uint64_t miso_attn_ragged_partials(uint32_t batch, uint32_t max_len) {
  return uint64_t{batch} * k::attn::kKvHeads * k::attn_ragged_splits(max_len) *
         (k::attn::kQHeads / k::attn::kKvHeads);
}

int miso_attn_decode_ragged(const float* q, const float* gate, const uint16_t* k_cache,
                            const uint16_t* v_cache, const uint64_t* kv_offsets,
                            const uint32_t* lens, uint32_t batch, uint32_t max_len, float* core,
                            float* part_m, float* part_l, float* part_o, void* stream) {
  if (any_bad(q, gate, k_cache, v_cache, core, part_o) || bad_scalars(part_m) ||
      bad_scalars(part_l) ||
      kv_offsets == nullptr || lens == nullptr)
    return fail("miso_attn_decode_ragged", kBadPtr);
  if (batch == 0)
    return fail("miso_attn_decode_ragged", "batch must be >= 1");
  if (max_len == 0)
    return fail("miso_attn_decode_ragged", "max_len must be >= 1");
  const unsigned s_max = k::attn_ragged_splits(max_len);
  const unsigned cus = device_cus();
  const k::AttnRaggedParams p{q,     gate,  as_half(k_cache), as_half(v_cache), kv_offsets,
                              lens,  core,  part_m,           part_l,           part_o,
                              batch, s_max, 0xFFFFFFFFu, k::attn_ragged_chunk(batch, max_len, cus)};
  const uint64_t items = uint64_t{batch} * k::attn::kKvHeads * s_max;
  if (items > 0x7FFFFFFFull)
    return fail("miso_attn_decode_ragged", "batch x splits too large for one grid");
  // One streaming workgroup per CU where the batch fits its item list; else one workgroup per
  // (sequence, KV head, split) slot. Same partials either way.
  const unsigned grid = static_cast<unsigned>(std::min<uint64_t>(cus, items));
  if (cus > 0 && k::attn_ragged_stream_fits(batch, s_max, grid))
    k::attn_ragged_stream_kernel<256><<<grid, 256, 0, as_stream(stream)>>>(p);
  else
    k::attn_ragged_split_kernel<256>
        <<<static_cast<unsigned>(items), 256, 0, as_stream(stream)>>>(p);
  int rc = launched("miso_attn_decode_ragged(split)");
  if (rc != 0)
    return rc;
  const unsigned tiles = batch * k::attn::kQHeads * (k::attn::kDim / 64);
  k::attn_ragged_combine_kernel<<<tiles, 64, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_decode_ragged(combine)");
}

int miso_attn_decode_paged(const float* q, const float* gate, const uint16_t* k_pages,
                           const uint16_t* v_pages, const int32_t* page_table, uint32_t max_pages,
                           uint32_t page_size, const uint32_t* lens, uint32_t batch,
                           uint32_t max_len, float* core, float* part_m, float* part_l,
                           float* part_o, void* stream) {
  if (any_bad(q, gate, k_pages, v_pages, core, part_o) || bad_scalars(part_m) ||
      bad_scalars(part_l) || page_table == nullptr || lens == nullptr)
    return fail("miso_attn_decode_paged", kBadPtr);
  if (batch == 0)
    return fail("miso_attn_decode_paged", "batch must be >= 1");
  if (max_len == 0)
    return fail("miso_attn_decode_paged", "max_len must be >= 1");
  if (max_pages == 0)
    return fail("miso_attn_decode_paged", "max_pages must be >= 1");
  if (page_size < 8 || page_size > 65536 || (page_size & (page_size - 1)) != 0)
    return fail("miso_attn_decode_paged", "page_size must be a power of two in [8, 65536]");
  if (uint64_t{max_pages} * page_size < max_len)
    return fail("miso_attn_decode_paged", "max_pages * page_size < max_len");
  const unsigned s_max = k::attn_ragged_splits(max_len);
  const uint64_t items = uint64_t{batch} * k::attn::kKvHeads * s_max;
  if (items > 0x7FFFFFFFull)
    return fail("miso_attn_decode_paged", "batch x splits too large for one grid");
  const unsigned cus = device_cus();
  const unsigned chunk = k::attn_ragged_chunk(batch, max_len, cus);
  const k::AttnPagedParams p{q,      as_half(k_pages), as_half(v_pages), page_table,
                             lens,   part_m,           part_l,           part_o,
                             batch,  s_max,            max_pages,
                             static_cast<unsigned>(__builtin_ctz(page_size)), chunk};
  // As the ragged decode: one streaming workgroup per CU where the batch fits its item list.
  const unsigned grid = static_cast<unsigned>(std::min<uint64_t>(cus, items));
  if (cus > 0 && k::attn_ragged_stream_fits(batch, s_max, grid))
    k::attn_paged_stream_kernel<256><<<grid, 256, 0, as_stream(stream)>>>(p);
  else
    k::attn_paged_split_kernel<256>
        <<<static_cast<unsigned>(items), 256, 0, as_stream(stream)>>>(p);
  int rc = launched("miso_attn_decode_paged(split)");
  if (rc != 0)
    return rc;
  // The merge reads only the partials, lens, gate and core of the ragged parameters.
  const k::AttnRaggedParams r{q,     gate,   nullptr, nullptr, nullptr,
                              lens,  core,   part_m,  part_l,  part_o,
                              batch, s_max,  k::attn_paged_len_cap(max_pages, p.log2_page), chunk};
  const unsigned tiles = batch * k::attn::kQHeads * (k::attn::kDim / 64);
  k::attn_ragged_combine_kernel<<<tiles, 64, 0, as_stream(stream)>>>(r);
  return launched("miso_attn_decode_paged(combine)");
}

int miso_attn_kv_encode_fp8(const uint16_t* k_cache, const uint16_t* v_cache, uint8_t* k8,
                            uint8_t* v8, float* k_scale, float* v_scale, uint32_t pos0, uint32_t n,
                            uint32_t max_ctx, void* stream) {
  if (n == 0)
    return 0;
  if (any_bad(k_cache, v_cache, k8, v8) || bad_scalars(k_scale) || bad_scalars(v_scale))
    return fail("miso_attn_kv_encode_fp8", kBadPtr);
  if (static_cast<uint64_t>(pos0) + n > max_ctx)
    return fail("miso_attn_kv_encode_fp8", "rows past max_ctx (pos0 + n > max_ctx)");
  const k::AttnKvFp8EncodeParams p{as_half(k_cache), as_half(v_cache), k8,  v8,     k_scale,
                                   v_scale,          pos0,             n,   max_ctx};
  const unsigned grid = n < 8192u ? n : 8192u;  // 4 rows per workgroup, grid-stride beyond
  k::attn_kv_fp8_encode_kernel<256><<<grid, 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_kv_encode_fp8");
}

int miso_attn_prep_fp8(const float* qg, const float* kp, const float* v, const float* q_norm,
                       const float* k_norm, const float* inv_freq, uint8_t* k8, uint8_t* v8,
                       float* k_scale, float* v_scale, float* q, uint32_t pos, uint32_t max_ctx,
                       float eps, void* stream) {
  if (any_bad(qg, kp, v, q_norm, k_norm, inv_freq, k8, v8, q) || bad_scalars(k_scale) ||
      bad_scalars(v_scale))
    return fail("miso_attn_prep_fp8", kBadPtr);
  if (pos >= max_ctx)
    return fail("miso_attn_prep_fp8", "KV cache is full (pos >= max_ctx)");
  const k::AttnPrepFp8Params p{qg, kp, v, q_norm, k_norm, inv_freq, k8, v8, k_scale, v_scale,
                               q,  pos, max_ctx, eps};
  k::attn_prep_fp8_kernel<256><<<18, 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prep_fp8");
}

int miso_attn_decode_fp8(const float* q, const float* qg, const uint8_t* k8, const uint8_t* v8,
                         const float* k_scale, const float* v_scale, float* core, float* part_m,
                         float* part_l, float* part_o, uint32_t len, uint32_t max_ctx,
                         uint32_t n_splits, void* stream) {
  if (any_bad(q, qg, k8, v8, core, part_o) || bad_scalars(k_scale) || bad_scalars(v_scale) ||
      bad_scalars(part_m) || bad_scalars(part_l))
    return fail("miso_attn_decode_fp8", kBadPtr);
  if (len == 0)
    return fail("miso_attn_decode_fp8", "len must be >= 1");
  if (len > max_ctx)
    return fail("miso_attn_decode_fp8", "len exceeds max_ctx");
  if (n_splits == 0)
    return fail("miso_attn_decode_fp8", "n_splits must be >= 1");
  const k::AttnSplitFp8Params p{q,      k8,     v8,     k_scale, v_scale, part_m,
                                part_l, part_o, len,    max_ctx, n_splits};
  k::attn_split_fp8_kernel<256><<<dim3(n_splits, 2), 256, 0, as_stream(stream)>>>(p);
  const int rc = launched("miso_attn_decode_fp8");
  if (rc != 0)
    return rc;
  return miso_attn_combine(part_m, part_l, part_o, qg, core, n_splits, stream);
}

int miso_attn_prep_batch_fp8(const float* qg, const float* kp, const float* v,
                             const float* q_norm, const float* k_norm, const float* inv_freq,
                             uint8_t* k8, uint8_t* v8, float* k_scale, float* v_scale, float* q,
                             uint32_t pos0, uint32_t max_ctx, float eps, uint32_t n,
                             uint32_t proj_stride, void* stream) {
  if (n == 0)
    return 0;
  if (any_bad(qg, kp, v, q_norm, k_norm, inv_freq, k8, v8, q) || bad_scalars(k_scale) ||
      bad_scalars(v_scale))
    return fail("miso_attn_prep_batch_fp8", kBadPtr);
  if (static_cast<uint64_t>(pos0) + n > max_ctx)
    return fail("miso_attn_prep_batch_fp8", "KV cache is full (pos0 + n > max_ctx)");
  if (proj_stride < 8192 + 1024)
    return fail("miso_attn_prep_batch_fp8",
                "proj_stride must cover [q+gate 8192 | k 512 | v 512]");
  const k::AttnPrepBatchFp8Params p{
      {qg, kp, v, q_norm, k_norm, inv_freq, k8, v8, k_scale, v_scale, q, pos0, max_ctx, eps},
      n,
      proj_stride};
  k::attn_prep_batch_fp8_kernel<256><<<n * 18, 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prep_batch_fp8");
}

int miso_attn_prefill_fp8(const float* q, const float* qg, const uint8_t* k8, const uint8_t* v8,
                          const float* k_scale, const float* v_scale, uint16_t* k_ws,
                          uint16_t* v_ws, float* core, uint32_t pos0, uint32_t n,
                          uint32_t max_ctx, uint32_t qg_stride, void* stream) {
  if (any_bad(q, qg, k8, v8, k_ws, v_ws, core) || bad_scalars(k_scale) || bad_scalars(v_scale))
    return fail("miso_attn_prefill_fp8", kBadPtr);
  if (n == 0)
    return fail("miso_attn_prefill_fp8", "n must be >= 1");
  if (static_cast<uint64_t>(pos0) + n > max_ctx)
    return fail("miso_attn_prefill_fp8", "KV cache is full (pos0 + n > max_ctx)");
  if (qg_stride < 8192 || qg_stride % 4 != 0)
    return fail("miso_attn_prefill_fp8", "qg_stride must be >= 8192 and a multiple of 4");
  const uint32_t rows = pos0 + n;
  const k::AttnKvFp8WidenParams w{k8,           v8, k_scale, v_scale, as_half(k_ws),
                                  as_half(v_ws), rows, max_ctx};
  const uint32_t wgrid = std::min<uint32_t>(rows, 4096);  // 4 rows per workgroup, grid-stride
  k::attn_kv_fp8_widen_kernel<256><<<wgrid, 256, 0, as_stream(stream)>>>(w);
  const int rc = launched("miso_attn_prefill_fp8");
  if (rc != 0)
    return rc;
  const k::AttnPrefillParams p{q, qg, as_half(k_ws), as_half(v_ws), core, pos0, n, rows,
                               qg_stride};
  k::attn_prefill_kernel<256><<<k::attn_prefill_items(n), 256, 0, as_stream(stream)>>>(p);
  return launched("miso_attn_prefill_fp8");
}

int miso_attn_q4k_gemv(const uint8_t* w, const float* x, float* y, uint32_t n_rows, uint32_t k,
                       int act_format, void* stream) {
  if (n_rows == 0)
    return 0;
  if (any_bad(w, x) || bad_scalars(y))
    return fail("miso_attn_q4k_gemv", kBadPtr);
  if (k != 2048 && k != 4096 && k != 8192)
    return fail("miso_attn_q4k_gemv", "k must be 2048, 4096 or 8192");
  if (act_format != 0 && act_format != 1)
    return fail("miso_attn_q4k_gemv", "act_format must be 0 (int8) or 1 (fp16)");
  const k::Q4kGemvParams p{w, x, y, n_rows};
  const hipStream_t st = as_stream(stream);
  if (act_format == 1) {
    if (k == 2048) q4k_gemv<k::ActFormat::Fp16, 2048>(p, st);
    else if (k == 4096) q4k_gemv<k::ActFormat::Fp16, 4096>(p, st);
    else q4k_gemv<k::ActFormat::Fp16, 8192>(p, st);
  } else {
    if (k == 2048) q4k_gemv<k::ActFormat::Int8, 2048>(p, st);
    else if (k == 4096) q4k_gemv<k::ActFormat::Int8, 4096>(p, st);
    else q4k_gemv<k::ActFormat::Int8, 8192>(p, st);
  }
  return launched("miso_attn_q4k_gemv");
}

int miso_attn_q6k_gemv(const uint8_t* w, const float* x, float* y, uint32_t n_rows, uint32_t k,
                       void* stream) {
  if (n_rows == 0)
    return 0;
  if (any_bad(w, x) || bad_scalars(y))
    return fail("miso_attn_q6k_gemv", kBadPtr);
  if (k != 2048 && k != 4096 && k != 8192)
    return fail("miso_attn_q6k_gemv", "k must be 2048, 4096 or 8192");
  const k::Q6kGemvParams p{w, x, y, n_rows};
  const hipStream_t st = as_stream(stream);
  if (k == 2048) q6k_gemv<2048>(p, st);
  else if (k == 4096) q6k_gemv<4096>(p, st);
  else q6k_gemv<8192>(p, st);
  return launched("miso_attn_q6k_gemv");
}

int miso_attn_q4k_q6k_gemv_pair(const uint8_t* w4, uint32_t n4, float* y4, const uint8_t* w6,
                                uint32_t n6, float* y6, const float* x, void* stream) {
  if (any_bad(w4, w6, x) || bad_scalars(y4) || bad_scalars(y6))
    return fail("miso_attn_q4k_q6k_gemv_pair", kBadPtr);
  if (n4 == 0 || n6 == 0)
    return fail("miso_attn_q4k_q6k_gemv_pair", "both row counts must be >= 1");
  // Logical grids sized for the attention's attn_q (8192 rows, 16 per Q4_K workgroup) and attn_v
  // (512 rows, 8 per Q6_K workgroup); other row counts grid-stride.
  constexpr unsigned kQ6Grid = 64, kQ4Grid = 512;
  const k::Q6kGemvParams p6{w6, x, y6, n6};
  const k::Q4kGemvParams p4{w4, x, y4, n4};
  k::mixed_gemv_kernel<1, kQ6Grid, kQ4Grid, 256>
      <<<kQ6Grid + kQ4Grid, 256, 0, as_stream(stream)>>>(p6, p4);
  return launched("miso_attn_q4k_q6k_gemv_pair");
}

int miso_attn_qkv_gemv(const uint8_t* wq, uint32_t nq, float* yq, const uint8_t* wk, uint32_t nk,
                       float* yk, const uint8_t* wv, uint32_t nv, float* yv, const float* x,
                       void* stream) {
  if (any_bad(wq, wk, wv, x) || bad_scalars(yq) || bad_scalars(yk) || bad_scalars(yv))
    return fail("miso_attn_qkv_gemv", kBadPtr);
  if (nq == 0 || nk == 0 || nv == 0)
    return fail("miso_attn_qkv_gemv", "all three row counts must be >= 1");
  // One launch; its logical grids are sized for 8192 / 512 / 512 rows (16 rows per Q4_K workgroup,
  // 8 per Q6_K), other counts grid-stride.
  const k::Q4kGemvParams pq{wq, x, yq, nq}, pk{wk, x, yk, nk};
  const k::Q6kGemvParams pv{wv, x, yv, nv};
  k::qkv_gemv_kernel<512, 32, 64, 256><<<512 + 32 + 64, 256, 0, as_stream(stream)>>>(pq, pk, pv);
  return launched("miso_attn_qkv_gemv");
}

int miso_attn_gemm_input(const float* x, uint16_t* xh, float* xs, uint32_t k, uint32_t n_tok,
                         void* stream) {
  if (n_tok == 0)
    return 0;
  if (any_bad(x, xh, xs))
    return fail("miso_attn_gemm_input", kBadPtr);
  if (k == 0 || k % 256 != 0)
    return fail("miso_attn_gemm_input", "k must be a positive multiple of 256");
  // One thread per 8 elements (the kernel grid-strides, so the reference's one-thread-per-group
  // grid also works, with four passes per thread).
  k::layer::gemm_input(x, k, n_tok, reinterpret_cast<_Float16*>(xh), xs, as_stream(stream));
  return launched("miso_attn_gemm_input");
}

int miso_attn_gemm(const uint8_t* w, int format, const uint16_t* xh, const float* xs, float* y,
                   uint32_t k, uint32_t n_rows, uint32_t n_tok, uint32_t ldy, void* stream) {
  if (n_tok == 0 || n_rows == 0)
    return 0;
  if (any_bad(w, xh) || (format == 0 && bad_ptr(xs)) || bad_scalars(y))
    return fail("miso_attn_gemm", kBadPtr);
  if (k == 0 || k % 256 != 0)
    return fail("miso_attn_gemm", "k must be a positive multiple of 256");
  if (ldy < n_rows)
    return fail("miso_attn_gemm", "ldy must be >= n_rows");
  const k::QGemmParams p{w, reinterpret_cast<const _Float16*>(xh), xs, y, k, n_rows, n_tok, ldy};
  const unsigned grid = k::qgemm_tiles(n_rows, n_tok);
  if (format == 0) {
    if (const unsigned big = k::qgemm_big_tiles(n_rows, n_tok))
      k::qgemm_q4k_big_kernel<><<<big, 256, 0, as_stream(stream)>>>(p);
    else
      k::qgemm_kernel<k::QFormat::Q4K><<<grid, 256, 0, as_stream(stream)>>>(p);
  } else if (format == 1)
    k::qgemm_kernel<k::QFormat::Q6K><<<grid, 256, 0, as_stream(stream)>>>(p);
  else
    return fail("miso_attn_gemm", "format must be 0 (Q4_K) or 1 (Q6_K)");
  return launched("miso_attn_gemm");
}

uint64_t miso_attn_layer_decode_ws(void) { return k::layer::decode_workspace_floats(); }

uint64_t miso_attn_layer_prefill_ws(uint32_t max_tok) {
  return k::layer::prefill_workspace_floats(max_tok);
}

uint64_t miso_attn_layer_decode_core(void) { return k::layer::decode_core_offset(); }

uint64_t miso_attn_layer_prefill_core(uint32_t max_tok) {
  return k::layer::prefill_core_offset(max_tok);
}

}  // extern "C"

namespace {

bool bad_matrix(const miso_attn_qmatrix& m) {
  return bad_ptr(m.w) || (m.format != 0 && m.format != 1);
}

// The C description of a layer as the wiring's (rejects null or misaligned pointers and unknown
// formats, then the shapes the projection layout needs).
const char* layer_view(const miso_attn_layer* in, k::layer::Weights& w) {
  if (in == nullptr)
    return kBadPtr;
  if (bad_matrix(in->q) || bad_matrix(in->k) || bad_matrix(in->v) || bad_matrix(in->o) ||
      any_bad(in->attn_norm, in->q_norm, in->k_norm, in->inv_freq))
    return "a layer pointer is NULL or not 16-byte aligned, or a format is not 0 or 1";
  auto view = [](const miso_attn_qmatrix& m) {
    return k::layer::Matrix{m.w, static_cast<k::layer::Format>(m.format), m.n_rows, m.k};
  };
  w = {view(in->q), view(in->k), view(in->v), view(in->o),
       in->attn_norm, in->q_norm, in->k_norm, in->inv_freq};
  return k::layer::check_weights(w);
}

int layer_result(const char* fn, const char* err) {
  return err != nullptr ? fail(fn, err) : launched(fn);
}

}  // namespace

extern "C" {

int miso_attn_layer_decode(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                           uint32_t len, uint32_t max_ctx, float* h, const float* delta, float* y,
                           float eps, float* ws, void* stream) {
  constexpr const char* fn = "miso_attn_layer_decode";
  k::layer::Weights w;
  if (const char* err = layer_view(layer, w))
    return fail(fn, err);
  if (any_bad(k_cache, v_cache, h, y, ws) || (delta != nullptr && bad_ptr(delta)))
    return fail(fn, kBadPtr);
  return layer_result(fn, k::layer::decode_step(w, as_half(k_cache), as_half(v_cache), len,
                                                max_ctx, h, delta, y, eps,
                                                k::layer::decode_workspace(ws),
                                                as_stream(stream)));
}

int miso_attn_layer_prefill(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                            uint32_t pos0, uint32_t n, uint32_t max_ctx, float* h,
                            const float* delta, float* y, float eps, float* ws, uint32_t max_tok,
                            void* stream) {
  constexpr const char* fn = "miso_attn_layer_prefill";
  if (n == 0)
    return 0;
  k::layer::Weights w;
  if (const char* err = layer_view(layer, w))
    return fail(fn, err);
  if (any_bad(k_cache, v_cache, h, y, ws) || (delta != nullptr && bad_ptr(delta)))
    return fail(fn, kBadPtr);
  return layer_result(fn, k::layer::prefill_step(w, as_half(k_cache), as_half(v_cache), pos0, n,
                                                 max_ctx, h, delta, y, eps,
                                                 k::layer::prefill_workspace(ws, max_tok),
                                                 max_tok, as_stream(stream)));
}

int miso_attn_layer_ingest(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                           uint32_t pos0, uint32_t n, uint32_t max_ctx, float* h,
                           const float* delta, float* y, float eps, float* decode_ws,
                           float* prefill_ws, uint32_t max_tok, uint32_t chunk, void* stream) {
  constexpr const char* fn = "miso_attn_layer_ingest";
  if (n == 0)
    return 0;
  k::layer::Weights w;
  if (const char* err = layer_view(layer, w))
    return fail(fn, err);
  if (any_bad(k_cache, v_cache, h, y, decode_ws) || (delta != nullptr && bad_ptr(delta)) ||
      (n >= k::layer::kPrefillMinTokens && bad_ptr(prefill_ws)))
    return fail(fn, kBadPtr);
  return layer_result(
      fn, k::layer::ingest(w, as_half(k_cache), as_half(v_cache), pos0, n, max_ctx, h, delta, y,
                           eps, k::layer::decode_workspace(decode_ws),
                           k::layer::prefill_workspace(prefill_ws, max_tok), max_tok, chunk,
                           as_stream(stream)));
}

}  // extern "C"
