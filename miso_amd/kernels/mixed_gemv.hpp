#pragma once

// Two independent projections of one activation vector in one launch: a Q6_K GEMV (attn_v) and a
// Q4_K GEMV with f16 activations (attn_q), K = 2048 -- the engine's gemv_pair
// (src/engine/weights.hip:286-307). Same names and template parameters as miso's
// kernels/mixed_gemv.hpp: mixed_gemv_op / mixed_gemv_kernel<Q6Rows, Q6Grid, Q4Grid, kBlock>; each
// operator keeps its own logical grid (Q6Grid / Q4Grid workgroups; the Q4_K operator takes two
// passes, 4 rows, per wave and step) and its own per-row arithmetic, so its outputs are
// bit-identical to its separate launch. The body is new.
//
// Workgroup order: stripes of one workgroup of the smaller logical grid followed by
// (larger / smaller) of the larger, so both kinds are in flight across the whole launch and each
// hides the other's memory latency.

#include "q4k_gemv.hpp"
#include "q6k_gemv.hpp"

namespace miso::kernels {

template <int Q6Rows, unsigned Q6Grid, unsigned Q4Grid, int kBlock = 256>
__device__ void mixed_gemv_op(const Q6kGemvParams& q6, const Q4kGemvParams& q4) {
  static_assert(Q6Grid > 0 && Q4Grid > 0, "both operators need workgroups");
  constexpr bool kQ6Larger = Q6Grid >= Q4Grid;
  constexpr unsigned kLarge = kQ6Larger ? Q6Grid : Q4Grid, kSmall = kQ6Larger ? Q4Grid : Q6Grid;
  static_assert(kLarge % kSmall == 0, "the larger logical grid is a multiple of the smaller");
  constexpr unsigned kPer = kLarge / kSmall, kStripe = kPer + 1;
  const unsigned stripe = blockIdx.x / kStripe, pos = blockIdx.x % kStripe;
  const bool small = pos == 0;  // uniform across the workgroup
  const unsigned logical = small ? stripe : stripe * kPer + pos - 1;
  if (small == kQ6Larger)  // this workgroup runs the Q4_K operator
    q4k_gemv_op<ActFormat::Fp16, 2048, kBlock, 2>(q4, 0, q4.n_rows, logical, Q4Grid);
  else
    q6k_gemv_op<2048, kBlock, Q6Rows>(q6, 0, q6.n_rows, logical, Q6Grid);
}

// Grid: Q6Grid + Q4Grid workgroups of kBlock threads.
template <int Q6Rows, unsigned Q6Grid, unsigned Q4Grid, int kBlock = 256>
__global__ void __launch_bounds__(kBlock) mixed_gemv_kernel(Q6kGemvParams q6, Q4kGemvParams q4) {
  mixed_gemv_op<Q6Rows, Q6Grid, Q4Grid, kBlock>(q6, q4);
}

// The attention's three input projections of one activation vector (K = 2048) in one launch: q
// and k (Q4_K, f16 activations) and v (Q6_K). No reference counterpart: the engine issues
// gemv_pair(q, v) then gemv(k) (src/engine/attention.hip:87-93). Workgroups [0, kVGrid) run v
// (one pass per wave, 8 rows per workgroup), the next kKGrid run k and the rest q (2 passes, 16
// rows per workgroup; k and q share one instantiation and so one LDS allocation), each operator on
// its own logical grid with its separate launch's per-row arithmetic (outputs bit-identical to the
// separate launches). v has the most arithmetic per byte, so its workgroups are dispatched first;
// at the engine's sizes all of them are resident at once.
template <unsigned kQGrid, unsigned kKGrid, unsigned kVGrid, int kBlock = 256>
__global__ void __launch_bounds__(kBlock) qkv_gemv_kernel(Q4kGemvParams q, Q4kGemvParams k,
                                                          Q6kGemvParams v) {
  const unsigned b = blockIdx.x;
  if (b < kVGrid)
    q6k_gemv_op<2048, kBlock, 1>(v, 0, v.n_rows, b, kVGrid);
  else if (b < kVGrid + kKGrid)
    q4k_gemv_op<ActFormat::Fp16, 2048, kBlock, 2>(k, 0, k.n_rows, b - kVGrid, kKGrid);
  else
    q4k_gemv_op<ActFormat::Fp16, 2048, kBlock, 2>(q, 0, q.n_rows, b - kVGrid - kKGrid, kQGrid);
}

}  // namespace miso::kernels
