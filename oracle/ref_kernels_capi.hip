// Test infrastructure: extern "C" launchers for the REFERENCE's attention kernels and its prefill
// GEMM activation prep (qgemm_act_kernel), compiled from the reference tree's own headers
// (include path set by oracle/Makefile, target `ref`). Used only by GPU tests, as a second
// checker next to the CPU oracle; never linked into the product.
//
// Launch shapes are the reference callers': split <<<dim3(n_splits, 2), 256>>>
// (src/engine/attention.hip:106), combine variants as tests/test_attn_splitk.hip:78-91 and
// src/engine/attention.hip:109, prefill <<<attn_prefill_items(n), 256>>> (:143-144), prep
// <<<18, 256>>> (:183), prep_batch <<<n * 18, 256>>> (:223); qgemm_act <<<ceil(groups / 256), 256>>>
// (src/engine/weights.hip:310-312).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "attention_decode.hpp"
#include "attention_prefill.hpp"
#include "qgemm.hpp"

namespace rk = miso::kernels;
using rk::attn::half_t;

namespace {

template <bool kPrepared, int kPipeline>
__global__ void ref_combine_range_kernel(rk::AttnCombineParams p, unsigned first, unsigned count) {
  rk::attn_combine_op<64, kPrepared, kPipeline>(p, first, count);
}

int done() { return static_cast<int>(hipGetLastError()); }

}  // namespace

extern "C" {

uint32_t ref_attn_n_splits(uint32_t len, uint32_t max_splits) {
  return rk::attn_n_splits(len, max_splits);
}

int ref_attn_split(const float* q, const uint16_t* kc, const uint16_t* vc, float* pm, float* pl,
                   float* po, uint32_t len, uint32_t max_ctx, uint32_t n_splits) {
  const rk::AttnSplitParams p{q,  reinterpret_cast<const half_t*>(kc),
                              reinterpret_cast<const half_t*>(vc), pm, pl, po, len, max_ctx,
                              n_splits};
  rk::attn_split_kernel<256><<<dim3(n_splits, 2), 256>>>(p);
  return done();
}

// variant: 0 = <256><<<16,256>>>, 1 = <64><<<64,64>>>, 2 = <64,true><<<64,64>>>,
// 3 = <64,true,4><<<64,64>>>.
int ref_attn_combine(int variant, const float* pm, const float* pl, const float* po,
                     const float* qg, float* core, uint32_t n_splits) {
  const rk::AttnCombineParams p{pm, pl, po, qg, core, n_splits};
  switch (variant) {
    case 0: rk::attn_combine_kernel<256><<<16, 256>>>(p); break;
    case 1: rk::attn_combine_kernel<64><<<64, 64>>>(p); break;
    case 2: rk::attn_combine_kernel<64, true><<<64, 64>>>(p); break;
    default: rk::attn_combine_kernel<64, true, 4><<<64, 64>>>(p); break;
  }
  return done();
}

int ref_attn_prefill(const float* q, const float* qg, const uint16_t* kc, const uint16_t* vc,
                     float* core, uint32_t pos0, uint32_t n, uint32_t max_ctx,
                     uint32_t qg_stride) {
  const rk::AttnPrefillParams p{q,    qg,   reinterpret_cast<const half_t*>(kc),
                                reinterpret_cast<const half_t*>(vc), core, pos0, n, max_ctx,
                                qg_stride};
  rk::attn_prefill_kernel<256><<<rk::attn_prefill_items(n), 256>>>(p);
  return done();
}

int ref_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm,
                  const float* k_norm, const float* inv_freq, uint16_t* kc, uint16_t* vc,
                  float* q, uint32_t pos, uint32_t max_ctx, float eps) {
  const rk::AttnPrepParams p{qg, k, v, q_norm, k_norm, inv_freq, reinterpret_cast<half_t*>(kc),
                             reinterpret_cast<half_t*>(vc), q, pos, max_ctx, eps};
  rk::attn_prep_kernel<256><<<18, 256>>>(p);
  return done();
}

int ref_attn_prep_batch(const float* qg, const float* k, const float* v, const float* q_norm,
                        const float* k_norm, const float* inv_freq, uint16_t* kc, uint16_t* vc,
                        float* q, uint32_t pos0, uint32_t max_ctx, float eps, uint32_t n,
                        uint32_t proj_stride) {
  const rk::AttnPrepBatchParams p{{qg, k, v, q_norm, k_norm, inv_freq,
                                   reinterpret_cast<half_t*>(kc), reinterpret_cast<half_t*>(vc),
                                   q, pos0, max_ctx, eps},
                                  n,
                                  proj_stride};
  rk::attn_prep_batch_kernel<256><<<n * 18, 256>>>(p);
  return done();
}

// The reference's GEMM input prep: x [n_tok][k] rounded to f16 (xh, as uint16 bits) and the sums
// of each 32-group of the rounded values (xs [n_tok][k / 32]).
int ref_qgemm_act(const float* x, uint16_t* xh, float* xs, uint32_t k, uint32_t n_tok) {
  const rk::QGemmActParams p{x, reinterpret_cast<_Float16*>(xh), xs, k, n_tok};
  const unsigned groups = n_tok * (k / 32);
  rk::qgemm_act_kernel<<<(groups + 255) / 256, 256>>>(p);
  return done();
}

}  // extern "C"
