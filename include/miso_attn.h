/*
 * miso_attn.h -- C ABI of the MI355X (gfx950) gated GQA softmax-attention library
 * (libmiso_attn.so).
 *
 * Every entry point launches the same kernels the C++ header API instantiates
 * (miso_amd/kernels/attention_decode.hpp, attention_prefill.hpp); the C ABI is the boundary a
 * non-C++ caller (ctypes, cgo, JNI) binds. Reference citations are relative to the reference
 * repository (penta2himajin/miso).
 *
 * Conventions
 *   - Pointers are device pointers (hipMalloc'd or equivalent). Every tensor pointer must be
 *     non-NULL and 16-byte aligned (the kernels move 16 bytes per lane), except part_m / part_l
 *     (4-byte aligned); a NULL or misaligned pointer is rejected with MISO_ATTN_EINVAL before
 *     any launch.
 *   - f16 buffers hold IEEE binary16 bit patterns (uint16_t).
 *   - Shapes are fixed by the model: 16 query heads, 2 KV heads, head_dim 256; the KV cache is
 *     [2][max_ctx][256] per tensor (K and V separate).
 *   - stream: a hipStream_t, or NULL for the null stream. Calls only enqueue; nothing
 *     synchronises the host.
 *   - Return value: 0 on success. A non-zero value is either a hipError_t from the launch or
 *     MISO_ATTN_EINVAL for arguments rejected on the host before any launch; the message is then
 *     available from miso_attn_last_error() (thread-local). The reference throws
 *     std::runtime_error in both situations (src/hip_util.hpp:12-17, src/engine/attention.hip:
 *     81-82, 110, 120-121, 145).
 */
#ifndef MISO_ATTN_H
#define MISO_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MISO_ATTN_EINVAL 0x4D41 /* host-side argument validation failed */

/* Message of the last failure on this thread ("" if none). */
const char* miso_attn_last_error(void);

/* Library / kernel-set version string. */
const char* miso_attn_version(void);

/* Split-count policy: replaces attn_n_splits(len, max_splits), kernels/attention_decode.hpp:92,
 * as used by src/engine/attention.hip:102. Returns 1 <= n <= max(max_splits, 1); 1 for len 0.
 * The MI355X policy differs from the reference's MI50 tuning (same contract). */
uint32_t miso_attn_n_splits(uint32_t len, uint32_t max_splits);

/* Prefill grid size: replaces attn_prefill_items(n), kernels/attention_prefill.hpp:54. */
uint32_t miso_attn_prefill_items(uint32_t n);

/* Decode prep: replaces attn_prep_kernel<256><<<18, 256, 0, stream>>>(AttnPrepParams{...}),
 * src/engine/attention.hip:97-100 (kernels/attention_decode.hpp:19-83). Per-head RMSNorm of the
 * 16 query heads (qg, gate half untouched) and 2 key heads, NEOX RoPE on dims [0, 64) at `pos`,
 * writes q [16][256] and appends K/V at position pos of the caches. Rejects pos >= max_ctx. */
int miso_attn_prep(const float* qg, const float* k, const float* v, const float* q_norm,
                   const float* k_norm, const float* inv_freq, uint16_t* k_cache,
                   uint16_t* v_cache, float* q, uint32_t pos, uint32_t max_ctx, float eps,
                   void* stream);

/* Batched prep for n tokens: replaces attn_prep_batch_kernel<256><<<n * 18, 256, 0, stream>>>,
 * src/engine/attention.hip:133-139 (kernels/attention_prefill.hpp:20-40). Token t reads qg/k/v
 * at t * proj_stride floats, writes q at t * 4096 floats and the cache at pos0 + t.
 * Rejects pos0 + n > max_ctx. */
int miso_attn_prep_batch(const float* qg, const float* k, const float* v, const float* q_norm,
                         const float* k_norm, const float* inv_freq, uint16_t* k_cache,
                         uint16_t* v_cache, float* q, uint32_t pos0, uint32_t max_ctx, float eps,
                         uint32_t n, uint32_t proj_stride, void* stream);

/* Split-K partials: replaces attn_split_kernel<256><<<dim3(n_splits, 2), 256, 0, stream>>>(
 * AttnSplitParams{...}), src/engine/attention.hip:103-106 and tests/test_attn_splitk.hip:125-134
 * (kernels/attention_decode.hpp:117-236). Writes part_m/part_l [2][n_splits][8] and part_o
 * [2][n_splits][8][256] for keys [0, len), at the reference's precision (f32 query, scores,
 * numerators and accumulation over the f16 cache), on the matrix cores: each f32 operand as an
 * exact f16 (hi, lo) pair. Rejects len == 0, len > max_ctx, n_splits == 0. */
int miso_attn_split(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                    float* part_m, float* part_l, float* part_o, uint32_t len, uint32_t max_ctx,
                    uint32_t n_splits, void* stream);

/* The same split and partials computed on wave64 VALU instead (attn_split_valu_kernel<256>,
 * v_fma_mix_f32: one f32 product per instruction). No reference counterpart: the measured
 * alternative to the matrix-core split, kept for comparison. Same arguments and rejections as
 * miso_attn_split. */
int miso_attn_split_valu(const float* q, const uint16_t* k_cache, const uint16_t* v_cache,
                         float* part_m, float* part_l, float* part_o, uint32_t len,
                         uint32_t max_ctx, uint32_t n_splits, void* stream);

/* LSE merge x sigmoid gate: replaces attn_combine_kernel<64, true, 4><<<64, 64, 0, stream>>>(
 * AttnCombineParams{...}), src/engine/attention.hip:107-109 (kernels/attention_decode.hpp:
 * 238-309). core [16][256] = merge of the partials x 1 / (1 + exp(-gate)), gate at qg[h*512 +
 * 256 + d]. Bit-identical to the reference's frozen merge order. Rejects n_splits == 0. */
int miso_attn_combine(const float* part_m, const float* part_l, const float* part_o,
                      const float* qg, float* core, uint32_t n_splits, void* stream);

/* The combine template variants and range form of the header API, launched as the reference's
 * test and bench do (tests/test_attn_splitk.hip:43-45,78-91; bench/attention/bench_combine.hip:
 * 40-46): variant 0 = attn_combine_kernel<256><<<16, 256>>>, 1 = <64><<<64, 64>>>,
 * 2 = <64, true><<<64, 64>>>, 3 = <64, true, 4><<<64, 64>>>. With count > 0 it instead launches
 * attn_combine_op<64, prepared, pipeline>(p, first, count) on <<<grid, 64>>> (variants 1-3;
 * tiles are h * 4 + dim / 64, 64 tiles in all). Every variant is bit-identical. */
int miso_attn_combine_variant(int variant, const float* part_m, const float* part_l,
                              const float* part_o, const float* qg, float* core,
                              uint32_t n_splits, uint32_t first, uint32_t count, uint32_t grid,
                              void* stream);

/* One decode step's attention: the split + combine pair of src/engine/attention.hip:102-109 in
 * one call, with n_splits chosen by the caller (miso_attn_n_splits(len, capacity)). The partial
 * buffers are caller-owned scratch of capacity >= n_splits. */
int miso_attn_decode(const float* q, const float* qg, const uint16_t* k_cache,
                     const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                     float* part_o, uint32_t len, uint32_t max_ctx, uint32_t n_splits,
                     void* stream);

/* The same decode step in ONE launch (attn_decode_fused_kernel, grid (n_splits, 2) x 256): each
 * split stores its partial agent-coherently and takes a ticket from its KV head's counter; the
 * last min(n_splits, 32) arrivals merge the head's 32 (head, 64-dimension) tiles in a fixed order
 * and apply the gate. No reference counterpart (the reference launches split then combine,
 * src/engine/attention.hip:103-109). sync: 4 uint32 of device memory, zero-filled once before
 * the first call; every call leaves it zero; calls that overlap on one sync buffer race.
 * Results are bit-equal from call to call and within the reference's rel-L2 gate (1e-5) of
 * miso_attn_decode's frozen merge order. On a device with <= 2 min(n_splits, 32) CUs (where
 * waiting mergers could hold every CU) it runs miso_attn_decode instead. Rejects what
 * miso_attn_decode rejects, n_splits > 128 and a NULL or misaligned sync. */
int miso_attn_decode_fused(const float* q, const float* qg, const uint16_t* k_cache,
                           const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                           float* part_o, uint32_t* sync, uint32_t len, uint32_t max_ctx,
                           uint32_t n_splits, void* stream);

/* The decode step with an f16 query and f16 softmax numerators (v_dot2_f32_f16, two products
 * per instruction): attn_split_f16q_kernel<256> then the combine of miso_attn_combine. No
 * reference counterpart -- the reference computes in f32 (kernels/attention_decode.hpp:150-221),
 * as miso_attn_split / miso_attn_decode do; this variant does half their VALU work at a per-head
 * relative L2 error of ~3e-4 instead of ~1e-6. Same arguments, scratch and rejections as
 * miso_attn_decode. */
int miso_attn_decode_f16q(const float* q, const float* qg, const uint16_t* k_cache,
                          const uint16_t* v_cache, float* core, float* part_m, float* part_l,
                          float* part_o, uint32_t len, uint32_t max_ctx, uint32_t n_splits,
                          void* stream);

/* miso_attn_decode without caller scratch (no reference counterpart; for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The split partials live in the library's own device array of
 * MISO_ATTN_NOALLOC_MAX_SPLITS splits (2,105,344 bytes per GPU, held until the process ends);
 * the call itself allocates nothing. Same kernels, arguments and results as miso_attn_decode
 * (bit-identical outputs). Rejects n_splits == 0 or n_splits > MISO_ATTN_NOALLOC_MAX_SPLITS, and
 * the arguments miso_attn_decode rejects. Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (different streams or host threads without ordering) race. */
#define MISO_ATTN_NOALLOC_MAX_SPLITS 128
int miso_attn_decode_noalloc(const float* q, const float* qg, const uint16_t* k_cache,
                             const uint16_t* v_cache, float* core, uint32_t len, uint32_t max_ctx,
                             uint32_t n_splits, void* stream);

/* Causal prefill: replaces attn_prefill_kernel<256><<<attn_prefill_items(n), 256, 0, stream>>>(
 * AttnPrefillParams{...}), src/engine/attention.hip:141-144 and tests/test_attn_splitk.hip:224-233
 * (kernels/attention_prefill.hpp:42-161). Tokens pos0 .. pos0 + n - 1; q [n][16][256] (unscaled),
 * gate at qg[t * qg_stride + h * 512 + 256 + d], keys [0, pos0 + n) already in the cache;
 * core [n][16][256]. Rejects n == 0, pos0 + n > max_ctx, qg_stride < 8192 or not a multiple of
 * 4 (the gate is read 16 bytes at a time). */
int miso_attn_prefill(const float* q, const float* qg, const uint16_t* k_cache,
                      const uint16_t* v_cache, float* core, uint32_t pos0, uint32_t n,
                      uint32_t max_ctx, uint32_t qg_stride, void* stream);

/* Balanced causal prefill (no reference counterpart: the reference launches one workgroup per
 * 16-token block, kernels/attention_prefill.hpp:42-161, so under the causal mask the last block
 * sets the time). Same arguments, contract and output as miso_attn_prefill (within the prefill
 * tolerance, not bitwise: the heavy blocks' keys are summed in two parts; bit-equal from call to
 * call). For n <= 2048 (16-token blocks) and for 3841 <= n <= 4096 (32-token blocks) token
 * block B-1-j of the B blocks is paired with block j and the pair's tiles are shared by two
 * workgroups (at most 256, one per CU); the two parts of a split block meet in `workspace`:
 * miso_attn_prefill_workspace_bytes(n) bytes of device memory, 16-byte aligned, zero-filled once
 * before its first use (every call leaves it reusable; one workspace of
 * miso_attn_prefill_workspace_bytes(4096) bytes serves every n). Calls that overlap on one
 * workspace race. For other n it runs miso_attn_prefill and the workspace is not used
 * (miso_attn_prefill_workspace_bytes returns 0). Rejects what miso_attn_prefill rejects and, for
 * the balanced sizes, a NULL or misaligned workspace or one smaller than required. */
uint64_t miso_attn_prefill_workspace_bytes(uint32_t n);
int miso_attn_prefill_ws(const float* q, const float* qg, const uint16_t* k_cache,
                         const uint16_t* v_cache, float* core, uint32_t pos0, uint32_t n,
                         uint32_t max_ctx, uint32_t qg_stride, void* workspace,
                         uint64_t workspace_bytes, void* stream);

/* Ragged batched decode (no reference counterpart: the reference is batch-1,
 * docs/decisions/ADR_002-build-scope-numerics-ops.md:14-18). batch sequences, one new token each:
 * q [batch][16][256] (unscaled), gate [batch][16][256], core [batch][16][256] = per-sequence
 * softmax(q K^T / 16) V x 1 / (1 + exp(-gate)). Sequence s has lens[s] keys stored contiguously
 * as K/V [2][lens[s]][256] (f16) starting kv_offsets[s] halves into k_cache / v_cache; lens and
 * kv_offsets are DEVICE arrays (not validated on the host: kv_offsets[s] must be a multiple of 8
 * and the K/V of every sequence inside the caches). max_len sizes the grid and the partial
 * scratch: every sequence is split into at most miso_attn_ragged_splits(max_len) spans (a longer sequence still gets all of
 * its keys, in longer spans). part_m/part_l need miso_attn_ragged_partials(batch, max_len) floats,
 * part_o 256 times that. A sequence with lens[s] == 0 yields core = 0. Rejects batch == 0 and
 * max_len == 0. */
uint32_t miso_attn_ragged_splits(uint32_t max_len);
uint64_t miso_attn_ragged_partials(uint32_t batch, uint32_t max_len);
/* Keys per span the ragged and paged decode use for this batch on the current device (no
 * reference counterpart): 1024 when 2 x batch x ceil(max_len / 1024) reaches four spans per CU,
 * else 512 (the scratch above is sized for 512, so it serves either). The same for both
 * layouts, so their outputs stay bit-identical. */
uint32_t miso_attn_ragged_chunk(uint32_t batch, uint32_t max_len);
int miso_attn_decode_ragged(const float* q, const float* gate, const uint16_t* k_cache,
                            const uint16_t* v_cache, const uint64_t* kv_offsets,
                            const uint32_t* lens, uint32_t batch, uint32_t max_len, float* core,
                            float* part_m, float* part_l, float* part_o, void* stream);

/* Paged batched decode (no reference counterpart; the reference's KV cache is one contiguous
 * [2][max_ctx][256] f16 buffer per layer, src/engine/attention.hpp:35-41). Same semantics, splits
 * and partial scratch as miso_attn_decode_ragged (and bit-identical outputs on the same keys), with
 * the keys in a pool of pages instead of contiguous per-sequence buffers: page g holds
 * [2 KV heads][page_size][256] f16 at g * 2 * page_size * 256 halves of k_pages / v_pages, and
 * sequence s's positions [j * page_size, (j + 1) * page_size) are in page
 * page_table[s * max_pages + j]. A sequence attends to min(lens[s], max_pages * page_size) keys:
 * a longer lens[s] is clamped to what its page-table row can address. page_table and lens are
 * DEVICE arrays (not validated on the host: every page id of a sequence's first
 * ceil(min(lens[s], max_pages * page_size) / page_size) entries must lie in the pool).
 * Rejects batch == 0, max_len == 0, max_pages == 0, page_size not a power of two in [8, 65536],
 * and max_pages * page_size < max_len. */
int miso_attn_decode_paged(const float* q, const float* gate, const uint16_t* k_pages,
                           const uint16_t* v_pages, const int32_t* page_table, uint32_t max_pages,
                           uint32_t page_size, const uint32_t* lens, uint32_t batch,
                           uint32_t max_len, float* core, float* part_m, float* part_l,
                           float* part_o, void* stream);

/* fp8 KV cache (no reference counterpart; the reference's cache is f16 [2][max_ctx][256],
 * src/engine/attention.hpp:35-41, kernels/attention_decode.hpp:26-27). Row (KV head, position)
 * is 256 OCP e4m3 codes in k8 / v8 [2][max_ctx][256] (uint8) plus one f32 power-of-two scale in
 * k_scale / v_scale [2][max_ctx]: value = scale * e4m3(code), scale = 2^(floor(log2 max|x|) - 7)
 * (rows whose max is below 2^-100 use 2^-107), codes rounded to nearest even, never saturated.
 * Inputs must be finite. k8 / v8 need 16-byte alignment, the scale arrays 4-byte alignment.
 *
 * miso_attn_kv_encode_fp8: rows [pos0, pos0 + n) of both KV heads of an f16 cache -> e4m3 rows
 * (n == 0 is a no-op). Rejects pos0 + n > max_ctx. */
int miso_attn_kv_encode_fp8(const uint16_t* k_cache, const uint16_t* v_cache, uint8_t* k8,
                            uint8_t* v8, float* k_scale, float* v_scale, uint32_t pos0, uint32_t n,
                            uint32_t max_ctx, void* stream);

/* miso_attn_prep with the token's K / V appended as e4m3 rows at position pos (q output and
 * arithmetic as miso_attn_prep). Rejects pos >= max_ctx. */
int miso_attn_prep_fp8(const float* qg, const float* k, const float* v, const float* q_norm,
                       const float* k_norm, const float* inv_freq, uint8_t* k8, uint8_t* v8,
                       float* k_scale, float* v_scale, float* q, uint32_t pos, uint32_t max_ctx,
                       float eps, void* stream);

/* miso_attn_decode over e4m3 rows: split-K partials (same spans and partial layout as
 * miso_attn_split) then miso_attn_combine. Same scratch sizes and rejections as
 * miso_attn_decode. */
int miso_attn_decode_fp8(const float* q, const float* qg, const uint8_t* k8, const uint8_t* v8,
                         const float* k_scale, const float* v_scale, float* core, float* part_m,
                         float* part_l, float* part_o, uint32_t len, uint32_t max_ctx,
                         uint32_t n_splits, void* stream);

/* miso_attn_prep_batch with the tokens' K / V appended as e4m3 rows at positions pos0 .. pos0 +
 * n - 1 (q output, layouts and rejections as miso_attn_prep_batch; every row equals the one
 * miso_attn_prep_fp8 writes for its token). n == 0 is a no-op. */
int miso_attn_prep_batch_fp8(const float* qg, const float* k, const float* v, const float* q_norm,
                             const float* k_norm, const float* inv_freq, uint8_t* k8, uint8_t* v8,
                             float* k_scale, float* v_scale, float* q, uint32_t pos0,
                             uint32_t max_ctx, float eps, uint32_t n, uint32_t proj_stride,
                             void* stream);

/* miso_attn_prefill over e4m3 rows: rows [0, pos0 + n) of both KV heads are widened to f16
 * (value = scale * e4m3(code), rounded to nearest even after saturating at +-65504) into the
 * caller's workspaces k_ws / v_ws, each 2 * (pos0 + n) * 256 binary16 values ([2][pos0 + n][256],
 * 16-byte aligned), then the f16 causal prefill runs over them. Layouts of q, qg, core and the
 * rejections as miso_attn_prefill. */
int miso_attn_prefill_fp8(const float* q, const float* qg, const uint8_t* k8, const uint8_t* v8,
                          const float* k_scale, const float* v_scale, uint16_t* k_ws,
                          uint16_t* v_ws, float* core, uint32_t pos0, uint32_t n,
                          uint32_t max_ctx, uint32_t qg_stride, void* stream);

/* Q4_K GEMV y = W x (the attention's Q4_K projections attn_q, attn_k, attn_output). Replaces the
 * launches of q4k_gemv_kernel<ActFormat, K, 256, R> in gemv() (src/engine/weights.hip:248-275,
 * kernels/q4k_gemv.hpp:196-239). w: n_rows rows of k / 256 Q4_K blocks in the r1 layout
 * (src/repack.hpp:14-19; 144 bytes per block, 16-byte aligned), x: k floats (16-byte aligned),
 * y: n_rows floats. act_format 1 converts x to f16 (the engine's choice), 0 to per-32 absmax
 * int8. n_rows == 0 is a no-op. Rejects k other than 2048, 4096, 8192 and other act_format
 * values. */
int miso_attn_q4k_gemv(const uint8_t* w, const float* x, float* y, uint32_t n_rows, uint32_t k,
                       int act_format, void* stream);

/* Q6_K GEMV y = W x with f16 activations (row f4: the attention's attn_v projection). Replaces the
 * launches of q6k_gemv_kernel<K, 256, R> in gemv() (src/engine/weights.hip:270-279,
 * kernels/q6k_gemv.hpp:85-131). w: n_rows Q6_K r1 rows (src/repack.hpp:25-28; k / 256 x 210
 * bytes rounded up to 16 per row, 16-byte aligned), x: k floats (16-byte aligned), y: n_rows
 * floats. n_rows == 0 is a no-op. Rejects k other than 2048, 4096, 8192. */
int miso_attn_q6k_gemv(const uint8_t* w, const float* x, float* y, uint32_t n_rows, uint32_t k,
                       void* stream);

/* The attention's q (Q4_K, f16 activations) and v (Q6_K) projections of one activation vector in
 * one launch, K = 2048. Replaces the mixed_gemv_kernel launch of gemv_pair()
 * (src/engine/weights.hip:286-307, kernels/mixed_gemv.hpp:12-30). w4: n4 Q4_K r1 rows -> y4;
 * w6: n6 Q6_K r1 rows -> y6; x: 2048 floats. Outputs are bit-identical to miso_attn_q4k_gemv
 * (act_format 1) and miso_attn_q6k_gemv on the same rows. Rejects n4 == 0 or n6 == 0. */
int miso_attn_q4k_q6k_gemv_pair(const uint8_t* w4, uint32_t n4, float* y4, const uint8_t* w6,
                                uint32_t n6, float* y6, const float* x, void* stream);

/* The attention's three input projections of one activation vector in one launch, K = 2048 (no
 * reference counterpart: the engine issues gemv_pair(q, v) then gemv(k),
 * src/engine/attention.hip:87-93). wq: nq Q4_K r1 rows -> yq, wk: nk Q4_K r1 rows -> yk (f16
 * activations), wv: nv Q6_K r1 rows -> yv; x: 2048 floats. Outputs are bit-identical to
 * miso_attn_q4k_gemv (act_format 1) and miso_attn_q6k_gemv. Rejects any row count of 0. */
int miso_attn_qkv_gemv(const uint8_t* wq, uint32_t nq, float* yq, const uint8_t* wk, uint32_t nk,
                       float* yk, const uint8_t* wv, uint32_t nv, float* yv, const float* x,
                       void* stream);

/* Prefill activations for the projection GEMMs: rounds x to f16 and sums every 32-element group of
 * the rounded values. Replaces gemm_input() (src/engine/weights.hip:306-314, the
 * qgemm_act_kernel launch of kernels/qgemm.hpp). x: n_tok x k floats, xh: n_tok x k binary16,
 * xs: n_tok x k / 32 floats, all 16-byte aligned. n_tok == 0 is a no-op. Rejects k == 0 or
 * k % 256 != 0 (the reference throws "gemm_input: chunk does not fit"). */
int miso_attn_gemm_input(const float* x, uint16_t* xh, float* xs, uint32_t k, uint32_t n_tok,
                         void* stream);

/* Prefill projection GEMM y[t * ldy + n] = sum_k W[n][k] xh[t][k] over n_rows quantized rows.
 * Replaces gemm() (src/engine/weights.hip:316-330, the qgemm_kernel<QFormat> launch of
 * kernels/qgemm.hpp). format 0: Q4_K r1 rows (144 bytes per 256 weights; uses xs), 1: Q6_K r1
 * rows (k / 256 x 210 bytes rounded up to 16). xh / xs as written by miso_attn_gemm_input for the
 * same k and n_tok; y: n_tok rows of stride ldy >= n_rows floats. n_tok == 0 or n_rows == 0 is a
 * no-op. Rejects k % 256 != 0, ldy < n_rows and any other format (the reference throws
 * "gemm: unsupported type"). */
int miso_attn_gemm(const uint8_t* w, int format, const uint16_t* xh, const float* xs, float* y,
                   uint32_t k, uint32_t n_rows, uint32_t n_tok, uint32_t ldy, void* stream);

/* ---------------------------------------------------------------------------------------------
 * One attention layer step: the host wiring of the engine's attention_decode / attention_prefill
 * (src/engine/attention.hip:76-148) over the entry points above, with the engine's sizing
 * retuned for one MI355X (the reference's values in brackets):
 *   MISO_ATTN_LAYER_MAX_SPLITS         decode split cap         [60,  src/engine/attention.hpp:46]
 *   MISO_ATTN_LAYER_MAX_CHUNK          prefill chunk, tokens    [512, src/engine/model.hpp:58]
 *   MISO_ATTN_LAYER_PREFILL_MIN_TOKENS prefill from this many   [8,   src/engine/model.hpp:80]
 * ------------------------------------------------------------------------------------------- */
#define MISO_ATTN_LAYER_MAX_SPLITS 128
#define MISO_ATTN_LAYER_MAX_CHUNK 4096
#define MISO_ATTN_LAYER_PREFILL_MIN_TOKENS 12

/* A quantized matrix (device): n_rows rows of k weights in the r1 layout of `format` (0: Q4_K, 144
 * bytes per 256 weights; 1: Q6_K, k / 256 x 210 bytes rounded up to 16 per row). */
typedef struct miso_attn_qmatrix {
  const uint8_t* w;
  int32_t format;
  uint32_t n_rows;
  uint32_t k;
} miso_attn_qmatrix;

/* One layer's weights (device), the engine's AttentionLayer (src/engine/attention.hpp:15-26) as
 * four separate matrices: q (8192 x 2048: per head 256 query then 256 gate rows), k and v
 * (512 x 2048), o (2048 x 4096); attn_norm [2048], q_norm / k_norm [256] (GGUF stores 1 + w),
 * inv_freq [32] (RoPE). */
typedef struct miso_attn_layer {
  miso_attn_qmatrix q, k, v, o;
  const float* attn_norm;
  const float* q_norm;
  const float* k_norm;
  const float* inv_freq;
} miso_attn_layer;

/* Device floats of the decode / prefill workspaces (the engine's AttentionScratch and
 * AttentionPrefillScratch, src/engine/attention.hpp:44-69), for chunks of up to max_tok tokens.
 * The prefill workspace ends with the balanced prefill's workspace (miso_attn_prefill_ws), which
 * chunks of up to 4096 tokens use: zero-fill it once when it is allocated (every call leaves its
 * pair counters zero). */
uint64_t miso_attn_layer_decode_ws(void);
uint64_t miso_attn_layer_prefill_ws(uint32_t max_tok);

/* Where each step leaves the attention output before the output projection, as a float offset
 * into its workspace: the engine's AttentionScratch::core (16 heads x 256 floats, the last decode
 * step's) and AttentionPrefillScratch::core ([n][16][256], the last prefill chunk's), which its
 * callers read (tests/test_attention.hip:68,104). */
uint64_t miso_attn_layer_decode_core(void);
uint64_t miso_attn_layer_prefill_core(uint32_t max_tok);

/* The token at position len: h += delta (delta may be NULL), y = o(Attention(RMSNorm(h))), K/V
 * appended at len. Replaces attention_decode() (src/engine/attention.hip:76-114): RMSNorm, the
 * q / k / v projections in one launch (Q4_K q and k, Q6_K v; other mixes one GEMV each), prep,
 * split + combine over len + 1 keys with miso_attn_n_splits(len + 1, MISO_ATTN_LAYER_MAX_SPLITS)
 * splits, output projection. h, y: 2048 floats; ws: miso_attn_layer_decode_ws() floats. Rejects
 * len >= max_ctx ("KV cache is full", as the reference) and matrices of other shapes. */
int miso_attn_layer_decode(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                           uint32_t len, uint32_t max_ctx, float* h, const float* delta, float* y,
                           float eps, float* ws, void* stream);

/* n consecutive tokens at pos0 (h, delta, y: [n][2048]). Replaces attention_prefill()
 * (src/engine/attention.hip:116-148): RMSNorm, the prefill GEMMs, batched prep, causal attention
 * over the cache up to each token, output GEMM. ws: miso_attn_layer_prefill_ws(max_tok) floats.
 * Rejects n > max_tok and pos0 + n > max_ctx. n == 0 is a no-op. */
int miso_attn_layer_prefill(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                            uint32_t pos0, uint32_t n, uint32_t max_ctx, float* h,
                            const float* delta, float* y, float eps, float* ws, uint32_t max_tok,
                            void* stream);

/* n tokens at pos0 with the engine's policy (src/engine/model.hip:130-175, for this layer):
 * n < MISO_ATTN_LAYER_PREFILL_MIN_TOKENS, one decode step per token; otherwise prefill chunks of
 * min(chunk ? chunk : MISO_ATTN_LAYER_MAX_CHUNK, max_tok) tokens. */
int miso_attn_layer_ingest(const miso_attn_layer* layer, uint16_t* k_cache, uint16_t* v_cache,
                           uint32_t pos0, uint32_t n, uint32_t max_ctx, float* h,
                           const float* delta, float* y, float eps, float* decode_ws,
                           float* prefill_ws, uint32_t max_tok, uint32_t chunk, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MISO_ATTN_H */
