/*
 * attn_oracle.c -- CPU oracle for the gated GQA softmax-attention path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load this library, and only as the checker: the product path (miso_amd/) never links,
 * loads or calls it.
 *
 * What it restates (paths relative to the reference repository, penta2himajin/miso):
 *   - oracle_decode_f64:   the FP64 host scalar reference of split-K decode,
 *                          tests/test_attn_splitk.hip:150-173
 *                          s_j = (q . k_j) / 16 in double, max-subtracted softmax,
 *                          o = sum_j p_j v_j / l, times 1 / (1 + exp(-gate)).
 *   - oracle_prefill_f64:  the FP64 host reference of causal prefill,
 *                          tests/test_attn_splitk.hip:237-266 (token t sees keys [0, pos0 + t]),
 *                          gate address as kernels/attention_prefill.hpp:149-150.
 *   - oracle_partials_f64: the (max, sum, unnormalised output) partial of one key span, as
 *                          written by kernels/attention_decode.hpp:224-228 (natural-log max of
 *                          the scaled scores; an empty span is (-inf, 0, 0)).
 *   - oracle_combine_f32:  the frozen FP32 merge order of tests/test_attn_splitk.hip:22-40
 *                          (M = max m_c; in split order w = exp(m_c - M), L += w l_c,
 *                          o += w o_c; core = o / L / (1 + exp(-gate))), with libm expf.
 *   - oracle_prep_f64:     per-head RMSNorm + NEOX RoPE + f16 KV append,
 *                          kernels/attention_decode.hpp:41-71, inv_freq as
 *                          src/engine/attention.hip:60-71.
 *   - oracle_ref_n_splits: the reference split-count policy, kernels/attention_decode.hpp:92-115.
 *   - oracle_ragged_f64:   oracle_decode_f64 per sequence with a dense [B][16][256] gate
 *                          (no reference function: the reference is batch-1).
 *   - oracle_e4m3_value / oracle_e4m3_encode / oracle_fp8_encode_rows / oracle_decode_fp8_f64:
 *                          the e4m3 KV-row format of miso_amd/kernels/attention_decode_fp8.hpp
 *                          and oracle_decode_f64 over its dequantized rows (no reference
 *                          function: the reference's cache is f16). The encoder is a search
 *                          for the nearest code, not the kernels' bit arithmetic.
 *   - oracle_q4k_scale_min / oracle_q4k_dequant: GGUF Q4_K, src/dequant.cpp:45-61,80-84;
 *                          oracle_q4k_mins: each element's dmin m (for the GEMM test's bound).
 *   - oracle_q4k_repack_r1: the r1 layout of the GPU GEMV, src/repack.cpp:9-25.
 *   - oracle_q4k_gemv_f64: y = W x in double over the dequantized rows, the reference of
 *                          tests/test_q4k_gemv.hip:80-90.
 *   - oracle_q6k_dequant / oracle_q6k_repack_r1 / oracle_q6k_gemv_f64: the same for Q6_K,
 *                          src/dequant.cpp:63-75, src/repack.cpp:53-74.
 *
 * Inputs come from a portable generator (splitmix64-seeded xoshiro256**, Box-Muller normals,
 * round-to-nearest-even binary16), so GPU tests and this oracle see bit-identical inputs on any
 * machine; the reference's own mt19937 + std::normal_distribution streams are not portable.
 *
 * Multi-threaded entry points split work over (token, head) rows with pthreads; the arithmetic
 * per row is identical to the single-threaded loops.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KQ 16
#define KKV 2
#define KD 256
#define KGROUP (KQ / KKV)

/* ------------------------------------------------------------------------------------------ */
/* Generator                                                                                   */
/* ------------------------------------------------------------------------------------------ */

uint64_t oracle_splitmix64(uint64_t* state) {
  uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

typedef struct {
  uint64_t s[4];
} xoshiro_t;

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static void xo_seed(xoshiro_t* g, uint64_t seed) {
  uint64_t sm = seed;
  for (int i = 0; i < 4; ++i) g->s[i] = oracle_splitmix64(&sm);
}

static inline uint64_t xo_next(xoshiro_t* g) {
  const uint64_t result = rotl64(g->s[1] * 5, 7) * 9;
  const uint64_t t = g->s[1] << 17;
  g->s[2] ^= g->s[0];
  g->s[3] ^= g->s[1];
  g->s[1] ^= g->s[2];
  g->s[0] ^= g->s[3];
  g->s[2] ^= t;
  g->s[3] = rotl64(g->s[3], 45);
  return result;
}

/* First n outputs of xoshiro256** seeded through splitmix64(seed); for known-answer tests. */
void oracle_xoshiro_stream(uint64_t seed, uint64_t* out, size_t n) {
  xoshiro_t g;
  xo_seed(&g, seed);
  for (size_t i = 0; i < n; ++i) out[i] = xo_next(&g);
}

/* First n outputs of xoshiro256** from an explicit state (known-answer tests of the core step). */
void oracle_xoshiro_raw(const uint64_t state[4], uint64_t* out, size_t n) {
  xoshiro_t g;
  for (int i = 0; i < 4; ++i) g.s[i] = state[i];
  for (size_t i = 0; i < n; ++i) out[i] = xo_next(&g);
}

/* Uniform double in (0, 1): 53 random bits, never 0. */
static inline double xo_unit(xoshiro_t* g) {
  return ((double)(xo_next(g) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

/* Box-Muller pair of N(0,1) values, computed in double then rounded to float. */
static inline void xo_normal2(xoshiro_t* g, float* a, float* b) {
  const double u1 = xo_unit(g), u2 = xo_unit(g);
  const double r = sqrt(-2.0 * log(u1));
  const double t = 6.283185307179586476925286766559 * u2;
  *a = (float)(r * cos(t));
  *b = (float)(r * sin(t));
}

/* out[i] = scale * N(0,1), stream (seed, i): element i is the (i % 2)-th value of pair i / 2. */
void oracle_fill_normal(uint64_t seed, float scale, float* out, size_t n) {
  xoshiro_t g;
  xo_seed(&g, seed);
  size_t i = 0;
  for (; i + 1 < n; i += 2) {
    float a, b;
    xo_normal2(&g, &a, &b);
    out[i] = scale * a;
    out[i + 1] = scale * b;
  }
  if (i < n) {
    float a, b;
    xo_normal2(&g, &a, &b);
    out[i] = scale * a;
  }
}

/* IEEE binary16, round to nearest even (subnormals, infinities and NaN handled). */
uint16_t oracle_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t ax = x & 0x7FFFFFFFu;
  if (ax >= 0x7F800000u) /* inf or nan */
    return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u | ((ax >> 13) & 0x3FFu) : 0u));
  if (ax >= 0x477FF000u) /* rounds to >= 65520: overflow to inf */
    return (uint16_t)(sign | 0x7C00u);
  if (ax < 0x38800000u) { /* below 2^-14: subnormal or zero */
    if (ax < 0x33000000u) return (uint16_t)sign; /* < 2^-25 rounds to zero (ties: 2^-25 -> 0) */
    const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
    const int e = (int)(ax >> 23) - 127;  /* -25 .. -15 */
    const int shift = -e - 14 + 13;       /* bits to drop to reach 2^-24 units */
    uint32_t q = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t h = ((ax - 0x38000000u) >> 13); /* rebias exponent 127 -> 15 */
  const uint32_t rem = ax & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  uint32_t x;
  if (e == 0) {
    if (m == 0) {
      x = sign;
    } else { /* subnormal: m * 2^-24 */
      const float v = (float)m * 5.9604644775390625e-8f;
      memcpy(&x, &v, 4);
      x |= sign;
    }
  } else if (e == 31) {
    x = sign | 0x7F800000u | (m << 13);
  } else {
    x = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &x, 4);
  return f;
}

void oracle_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

/* binary16 of N(0,1) values: the normal stream of oracle_fill_normal, rounded. */
void oracle_fill_normal_f16(uint64_t seed, uint16_t* out, size_t n) {
  xoshiro_t g;
  xo_seed(&g, seed);
  size_t i = 0;
  for (; i + 1 < n; i += 2) {
    float a, b;
    xo_normal2(&g, &a, &b);
    out[i] = oracle_f32_to_f16(a);
    out[i + 1] = oracle_f32_to_f16(b);
  }
  if (i < n) {
    float a, b;
    xo_normal2(&g, &a, &b);
    out[i] = oracle_f32_to_f16(a);
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Thread pool helper                                                                          */
/* ------------------------------------------------------------------------------------------ */

typedef void (*row_fn)(void* ctx, size_t row);
typedef struct {
  row_fn fn;
  void* ctx;
  size_t rows;
  int threads, tid;
} par_arg_t;

static void* par_worker(void* p) {
  par_arg_t* a = (par_arg_t*)p;
  for (size_t r = (size_t)a->tid; r < a->rows; r += (size_t)a->threads) a->fn(a->ctx, r);
  return NULL;
}

static void parallel_rows(row_fn fn, void* ctx, size_t rows, int threads) {
  if (threads <= 1 || rows <= 1) {
    for (size_t r = 0; r < rows; ++r) fn(ctx, r);
    return;
  }
  if ((size_t)threads > rows) threads = (int)rows;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)threads);
  par_arg_t* args = (par_arg_t*)malloc(sizeof(par_arg_t) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    args[t].fn = fn, args[t].ctx = ctx, args[t].rows = rows, args[t].threads = threads;
    args[t].tid = t;
    pthread_create(&th[t], NULL, par_worker, &args[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(th[t], NULL);
  free(th);
  free(args);
}

/* ------------------------------------------------------------------------------------------ */
/* One (query row, head): softmax(q K^T / 16) V / (1 + exp(-gate))                             */
/* ------------------------------------------------------------------------------------------ */

/* K, V: the KV head's rows (row stride KD halves); seen: keys [0, seen). gate: KD floats.
 * out: KD doubles. scratch: seen doubles. Follows tests/test_attn_splitk.hip:153-172. */
static void attend_row(const float* q, const float* gate, const uint16_t* K, const uint16_t* V,
                       size_t seen, double* s, double* out) {
  double mx = -1e300;
  for (size_t j = 0; j < seen; ++j) {
    const uint16_t* kr = K + j * KD;
    double d = 0;
    for (int e = 0; e < KD; ++e) d += (double)q[e] * (double)oracle_f16_to_f32(kr[e]);
    s[j] = d / 16.0;
    if (s[j] > mx) mx = s[j];
  }
  double l = 0;
  for (size_t j = 0; j < seen; ++j) {
    s[j] = exp(s[j] - mx);
    l += s[j];
  }
  double o[KD];
  for (int e = 0; e < KD; ++e) o[e] = 0;
  for (size_t j = 0; j < seen; ++j) {
    const uint16_t* vr = V + j * KD;
    const double pj = s[j];
    for (int e = 0; e < KD; ++e) o[e] += pj * (double)oracle_f16_to_f32(vr[e]);
  }
  for (int e = 0; e < KD; ++e) out[e] = o[e] / l / (1.0 + exp(-(double)gate[e]));
}

/* ------------------------------------------------------------------------------------------ */
/* Decode                                                                                      */
/* ------------------------------------------------------------------------------------------ */

typedef struct {
  const float* q;          /* [16][256] */
  const float* gate;       /* base of the gate rows */
  size_t gate_head_stride; /* floats between heads' gate rows */
  const uint16_t* kc;      /* [2][max_ctx][256] */
  const uint16_t* vc;
  size_t len, max_ctx;
  double* out; /* [16][256] */
} decode_ctx_t;

static void decode_row(void* p, size_t h) {
  decode_ctx_t* c = (decode_ctx_t*)p;
  const size_t kvh = h / KGROUP;
  double* s = (double*)malloc(sizeof(double) * (c->len ? c->len : 1));
  attend_row(c->q + h * KD, c->gate + h * c->gate_head_stride, c->kc + kvh * c->max_ctx * KD,
             c->vc + kvh * c->max_ctx * KD, c->len, s, c->out + h * KD);
  free(s);
}

/* qg: [16][512] (gate half at h*512 + 256), as AttnCombineParams::qg. */
void oracle_decode_f64(const float* q, const float* qg, const uint16_t* kc, const uint16_t* vc,
                       uint32_t len, uint32_t max_ctx, double* out, int threads) {
  decode_ctx_t c = {q, qg + KD, 2 * KD, kc, vc, len, max_ctx, out};
  parallel_rows(decode_row, &c, KQ, threads);
}

/* Ragged batch: q [B][16][256], gate [B][16][256], per-sequence K/V [2][L_s][256] at
 * kv_off[s] halves into kc / vc, out [B][16][256]. Rows are (sequence, head). */
typedef struct {
  const float* q;
  const float* gate;
  const uint16_t* kc;
  const uint16_t* vc;
  const uint64_t* kv_off;
  const uint32_t* lens;
  double* out;
} ragged_ctx_t;

static void ragged_row(void* p, size_t row) {
  ragged_ctx_t* c = (ragged_ctx_t*)p;
  const size_t sq = row / KQ, h = row % KQ, kvh = h / KGROUP, L = c->lens[sq];
  double* s = (double*)malloc(sizeof(double) * (L ? L : 1));
  const uint16_t* K = c->kc + c->kv_off[sq] + kvh * L * KD;
  const uint16_t* V = c->vc + c->kv_off[sq] + kvh * L * KD;
  attend_row(c->q + row * KD, c->gate + row * KD, K, V, L, s, c->out + row * KD);
  free(s);
}

void oracle_ragged_f64(const float* q, const float* gate, const uint16_t* kc, const uint16_t* vc,
                       const uint64_t* kv_off, const uint32_t* lens, uint32_t batch, double* out,
                       int threads) {
  ragged_ctx_t c = {q, gate, kc, vc, kv_off, lens, out};
  parallel_rows(ragged_row, &c, (size_t)batch * KQ, threads);
}

/* ------------------------------------------------------------------------------------------ */
/* Prefill                                                                                     */
/* ------------------------------------------------------------------------------------------ */

typedef struct {
  const float* q;  /* [n][16][256] */
  const float* qg; /* token-major, stride qg_stride; gate at t*qg_stride + h*512 + 256 */
  size_t qg_stride;
  const uint16_t* kc;
  const uint16_t* vc;
  size_t pos0, max_ctx;
  const uint32_t* tokens; /* token indices to evaluate */
  double* out;            /* [n_tokens][16][256] */
} prefill_ctx_t;

static void prefill_row(void* p, size_t row) {
  prefill_ctx_t* c = (prefill_ctx_t*)p;
  const size_t i = row / KQ, h = row % KQ, kvh = h / KGROUP;
  const size_t t = c->tokens[i], seen = c->pos0 + t + 1;
  double* s = (double*)malloc(sizeof(double) * seen);
  attend_row(c->q + (t * KQ + h) * KD, c->qg + t * c->qg_stride + h * 2 * KD + KD,
             c->kc + kvh * c->max_ctx * KD, c->vc + kvh * c->max_ctx * KD, seen, s,
             c->out + row * KD);
  free(s);
}

void oracle_prefill_f64(const float* q, const float* qg, uint32_t qg_stride, const uint16_t* kc,
                        const uint16_t* vc, uint32_t pos0, uint32_t max_ctx,
                        const uint32_t* tokens, uint32_t n_tokens, double* out, int threads) {
  prefill_ctx_t c = {q, qg, qg_stride, kc, vc, pos0, max_ctx, tokens, out};
  parallel_rows(prefill_row, &c, (size_t)n_tokens * KQ, threads);
}

/* ------------------------------------------------------------------------------------------ */
/* Split partials and the frozen FP32 combine                                                  */
/* ------------------------------------------------------------------------------------------ */

/* Partial of keys [j0, j1) for the 8 query heads of KV head kvh: m[8] (natural-log max of
 * q.k/16), l[8] = sum exp(s - m), o[8][256] = sum exp(s - m) v. Empty span: (-inf, 0, 0). */
void oracle_partials_f64(const float* q, const uint16_t* kc, const uint16_t* vc, uint32_t kvh,
                         uint32_t max_ctx, uint32_t j0, uint32_t j1, double* m, double* l,
                         double* o) {
  for (int h = 0; h < KGROUP; ++h) {
    const float* qq = q + ((size_t)kvh * KGROUP + h) * KD;
    double* oo = o + (size_t)h * KD;
    for (int e = 0; e < KD; ++e) oo[e] = 0;
    if (j1 <= j0) {
      m[h] = -INFINITY, l[h] = 0;
      continue;
    }
    double mx = -1e300;
    double* s = (double*)malloc(sizeof(double) * (j1 - j0));
    for (uint32_t j = j0; j < j1; ++j) {
      const uint16_t* kr = kc + ((size_t)kvh * max_ctx + j) * KD;
      double d = 0;
      for (int e = 0; e < KD; ++e) d += (double)qq[e] * (double)oracle_f16_to_f32(kr[e]);
      s[j - j0] = d / 16.0;
      if (s[j - j0] > mx) mx = s[j - j0];
    }
    double sum = 0;
    for (uint32_t j = j0; j < j1; ++j) {
      const double pj = exp(s[j - j0] - mx);
      sum += pj;
      const uint16_t* vr = vc + ((size_t)kvh * max_ctx + j) * KD;
      for (int e = 0; e < KD; ++e) oo[e] += pj * (double)oracle_f16_to_f32(vr[e]);
    }
    m[h] = mx, l[h] = sum;
    free(s);
  }
}

/* The frozen merge order, FP32 arithmetic with libm expf and fmaf for the two accumulations.
 * part_*: [2][n_splits][8](x256); qg [16][512]; core [16][256]. */
void oracle_combine_f32(const float* part_m, const float* part_l, const float* part_o,
                        const float* qg, uint32_t n_splits, float* core) {
  for (int h = 0; h < KQ; ++h) {
    const int kvh = h / KGROUP, hl = h % KGROUP;
    for (int d = 0; d < KD; ++d) {
      float M = -INFINITY;
      for (uint32_t c = 0; c < n_splits; ++c)
        M = fmaxf(M, part_m[((size_t)kvh * n_splits + c) * KGROUP + hl]);
      float L = 0, o = 0;
      for (uint32_t c = 0; c < n_splits; ++c) {
        const size_t i = ((size_t)kvh * n_splits + c) * KGROUP + hl;
        const float w = expf(part_m[i] - M);
        L = fmaf(w, part_l[i], L);
        o = fmaf(w, part_o[i * KD + d], o);
      }
      const float gate = qg[h * 2 * KD + KD + d];
      core[h * KD + d] = o / L / (1.0f + expf(-gate));
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* Prep: per-head RMSNorm + NEOX RoPE on the first 64 dims + KV append                         */
/* ------------------------------------------------------------------------------------------ */

/* inv_freq[i] = 1 / base^(2i/64) in FP32, as src/engine/attention.hip:60-71. */
void oracle_inv_freq(float base, float* inv /* [32] */) {
  for (int i = 0; i < 32; ++i) inv[i] = 1.0f / powf(base, (float)(2 * i) / 64.0f);
}

/* One token: qg [16][512], k [2][256], v [2][256] (floats), weights q_norm/k_norm [256],
 * inv_freq [32]. Outputs: q_out [16][256] (double), k_out/v_out [2][256] as binary16. */
void oracle_prep_f64(const float* qg, const float* k, const float* v, const float* q_norm,
                     const float* k_norm, const float* inv_freq, uint32_t pos, float eps,
                     double* q_out, uint16_t* k_out, uint16_t* v_out) {
  for (int head = 0; head < KQ + KKV; ++head) {
    const int is_q = head < KQ, kvh = head - KQ;
    const float* x = is_q ? qg + head * 2 * KD : k + kvh * KD;
    const float* w = is_q ? q_norm : k_norm;
    double ss = 0;
    for (int d = 0; d < KD; ++d) ss += (double)x[d] * (double)x[d];
    const double r = 1.0 / sqrt(ss / KD + (double)eps);
    double y[KD];
    for (int d = 0; d < KD; ++d) y[d] = (double)x[d] * r * (double)w[d];
    double z[KD];
    memcpy(z, y, sizeof(z));
    for (int i = 0; i < 32; ++i) {
      /* theta as the device computes it: float(pos) * inv_freq[i], rounded to float. */
      const double th = (double)((float)pos * inv_freq[i]);
      const double c = cos(th), s = sin(th);
      z[i] = y[i] * c - y[i + 32] * s;
      z[i + 32] = y[i + 32] * c + y[i] * s;
    }
    if (is_q) {
      for (int d = 0; d < KD; ++d) q_out[head * KD + d] = z[d];
    } else {
      for (int d = 0; d < KD; ++d) {
        k_out[kvh * KD + d] = oracle_f32_to_f16((float)z[d]);
        v_out[kvh * KD + d] = oracle_f32_to_f16(v[kvh * KD + d]);
      }
    }
  }
}

/* ------------------------------------------------------------------------------------------ */
/* The reference split-count policy (kernels/attention_decode.hpp:92-115)                      */
/* ------------------------------------------------------------------------------------------ */

uint32_t oracle_ref_n_splits(uint32_t len, uint32_t max_splits) {
  const uint32_t sub = 32;
  const uint32_t subs = (len + sub - 1) / sub;
  if (subs == 0) return 1;
  uint32_t per = 6, n = (subs + per - 1) / per;
  if (n > max_splits) {
    per = (subs + max_splits - 1) / max_splits;
    n = (subs + per - 1) / per;
  } else if (n < 16 && max_splits >= 16) {
    const uint32_t target = subs < 16 ? subs : 16;
    if (n < target) {
      per = (subs + target - 1) / target;
      n = (subs + per - 1) / per;
    }
  }
  return n;
}

/* ------------------------------------------------------------------------------------------ */
/* e4m3 KV rows (no reference counterpart: the reference's cache is f16,                       */
/* src/engine/attention.hpp:35-41). Restates the format documented in                          */
/* miso_amd/kernels/attention_decode_fp8.hpp: value = scale * e4m3(code), OCP e4m3 (bias 7,    */
/* subnormal step 2^-9, max 448), scale = 2^(E - 7) with E = floor(log2 max|x|) (>= -100).     */
/* ------------------------------------------------------------------------------------------ */

/* Value of an e4m3 code from its fields (0x7F / 0xFF are NaN). */
double oracle_e4m3_value(uint8_t c) {
  const int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7) return NAN;
  const double v = e ? ldexp(1.0 + m / 8.0, e - 7) : ldexp(m / 8.0, -6);
  return s ? -v : v;
}

/* Round-to-nearest-even e4m3 code of y, |y| < 256, by search: the representable magnitude
 * nearest to |y|, ties to the even code (the one with a clear lowest mantissa bit). */
uint8_t oracle_e4m3_encode(float y) {
  const double a = fabs((double)y);
  int best = 0;
  double best_err = INFINITY;
  for (int c = 0; c <= 0x78; ++c) {
    const double err = fabs(oracle_e4m3_value((uint8_t)c) - a);
    if (err < best_err || (err == best_err && (c & 1) == 0)) best = c, best_err = err;
  }
  return (uint8_t)(best | (signbit(y) ? 0x80 : 0));
}

/* Rows of 256 floats -> codes and power-of-two scales. */
void oracle_fp8_encode_rows(const float* x, size_t rows, uint8_t* codes, float* scales) {
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * KD;
    float amax = 0;
    for (int d = 0; d < KD; ++d)
      if (fabsf(xr[d]) > amax) amax = fabsf(xr[d]);
    int e = -100;
    if (amax > 0) {
      int ex;
      frexpf(amax, &ex); /* amax = f 2^ex, f in [0.5, 1): floor(log2 amax) = ex - 1 */
      if (ex - 1 > e) e = ex - 1;
    }
    const float inv = ldexpf(1.0f, 7 - e);
    for (int d = 0; d < KD; ++d) codes[r * KD + d] = oracle_e4m3_encode(xr[d] * inv);
    scales[r] = ldexpf(1.0f, e - 7);
  }
}

/* attend_row over e4m3 rows: K / V row j is scale[j] * e4m3(code[j][.]), in double. */
static void attend_row_fp8(const float* q, const float* gate, const uint8_t* K, const uint8_t* V,
                           const float* ks, const float* vs, size_t seen, double* s,
                           double* out) {
  double lut[256];
  for (int c = 0; c < 256; ++c) lut[c] = oracle_e4m3_value((uint8_t)c);
  double mx = -1e300;
  for (size_t j = 0; j < seen; ++j) {
    const uint8_t* kr = K + j * KD;
    double d = 0;
    for (int e = 0; e < KD; ++e) d += (double)q[e] * lut[kr[e]];
    s[j] = d * (double)ks[j] / 16.0;
    if (s[j] > mx) mx = s[j];
  }
  double l = 0;
  for (size_t j = 0; j < seen; ++j) {
    s[j] = exp(s[j] - mx);
    l += s[j];
  }
  double o[KD];
  for (int e = 0; e < KD; ++e) o[e] = 0;
  for (size_t j = 0; j < seen; ++j) {
    const uint8_t* vr = V + j * KD;
    const double pj = s[j] * (double)vs[j];
    for (int e = 0; e < KD; ++e) o[e] += pj * lut[vr[e]];
  }
  for (int e = 0; e < KD; ++e) out[e] = o[e] / l / (1.0 + exp(-(double)gate[e]));
}

typedef struct {
  const float* q;
  const float* qg;
  const uint8_t* k8;
  const uint8_t* v8;
  const float* ks;
  const float* vs;
  size_t len, max_ctx;
  double* out;
} decode_fp8_ctx_t;

static void decode_fp8_row(void* p, size_t h) {
  decode_fp8_ctx_t* c = (decode_fp8_ctx_t*)p;
  const size_t kvh = h / KGROUP, base = kvh * c->max_ctx;
  double* s = (double*)malloc(sizeof(double) * (c->len ? c->len : 1));
  attend_row_fp8(c->q + h * KD, c->qg + h * 2 * KD + KD, c->k8 + base * KD, c->v8 + base * KD,
                 c->ks + base, c->vs + base, c->len, s, c->out + h * KD);
  free(s);
}

/* oracle_decode_f64 over e4m3 rows: k8 / v8 [2][max_ctx][256], ks / vs [2][max_ctx]. */
void oracle_decode_fp8_f64(const float* q, const float* qg, const uint8_t* k8, const uint8_t* v8,
                           const float* ks, const float* vs, uint32_t len, uint32_t max_ctx,
                           double* out, int threads) {
  decode_fp8_ctx_t c = {q, qg, k8, v8, ks, vs, len, max_ctx, out};
  parallel_rows(decode_fp8_row, &c, KQ, threads);
}

/* ------------------------------------------------------------------------------------------ */
/* Q4_K weights of the attention's projections (row f4: attn_q / attn_k / attn_output).       */
/* GGUF Q4_K block (144 bytes): f16 d, f16 dmin, 12 bytes of packed 6-bit (scale, min) pairs  */
/* for 8 sub-blocks of 32, 128 bytes of nibbles (sub-block 2g: low nibbles of bytes 32g..+31, */
/* 2g + 1: their high nibbles). w = d sc q - dmin m.                                            */
/* ------------------------------------------------------------------------------------------ */

static float f16_at(const uint8_t* p) { return oracle_f16_to_f32((uint16_t)(p[0] | p[1] << 8)); }

/* 6-bit scale and min of sub-block j, src/dequant.cpp:80-84. */
void oracle_q4k_scale_min(const uint8_t* block, int j, uint8_t* sc, uint8_t* m) {
  const uint8_t* s = block + 4;
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (uint8_t)((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4));
    *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
  }
}

/* Dequantize n_blocks GGUF Q4_K blocks to 256 floats each, in f32 as src/dequant.cpp:45-61
 * (dj = d sc, mj = dmin m, y = dj q - mj). ds (optional): d sc of each element's sub-block. */
void oracle_q4k_dequant(const uint8_t* blocks, size_t n_blocks, float* out, float* ds) {
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* blk = blocks + b * 144;
    const float d = f16_at(blk), dmin = f16_at(blk + 2);
    for (int j = 0; j < 8; ++j) {
      uint8_t sc, m;
      oracle_q4k_scale_min(blk, j, &sc, &m);
      const float dj = d * (float)sc, mj = dmin * (float)m;
      const uint8_t* q = blk + 16 + 32 * (j / 2);
      for (int l = 0; l < 32; ++l) {
        const int v = (q[l] >> (4 * (j % 2))) & 15;
        out[b * 256 + 32 * j + l] = dj * (float)v - mj;
        if (ds) ds[b * 256 + 32 * j + l] = dj;
      }
    }
  }
}

/* dmin m of each element's sub-block for n_blocks GGUF Q4_K blocks (the magnitude of a weight's
 * min term, one of the two parts of the per-element bound of tests/test_qgemm.hip:46-53). */
void oracle_q4k_mins(const uint8_t* blocks, size_t n_blocks, float* dm) {
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* blk = blocks + b * 144;
    const float dmin = f16_at(blk + 2);
    for (int j = 0; j < 8; ++j) {
      uint8_t sc, m;
      oracle_q4k_scale_min(blk, j, &sc, &m);
      for (int l = 0; l < 32; ++l) dm[b * 256 + 32 * j + l] = dmin * (float)m;
    }
  }
}

/* GGUF -> r1 (src/repack.cpp:9-25): bytes 4..15 become, per nibble group g, the 24-bit
 * little-endian value sc[2g] | m[2g] << 6 | sc[2g+1] << 12 | m[2g+1] << 18 at byte 4 + 3 g. */
void oracle_q4k_repack_r1(const uint8_t* src, size_t n_blocks, uint8_t* dst) {
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* s = src + b * 144;
    uint8_t* d = dst + b * 144;
    memcpy(d, s, 144);
    for (int g = 0; g < 4; ++g) {
      uint8_t sc0, m0, sc1, m1;
      oracle_q4k_scale_min(s, 2 * g, &sc0, &m0);
      oracle_q4k_scale_min(s, 2 * g + 1, &sc1, &m1);
      const uint32_t v =
          (uint32_t)sc0 | (uint32_t)m0 << 6 | (uint32_t)sc1 << 12 | (uint32_t)m1 << 18;
      for (int i = 0; i < 3; ++i) d[4 + 3 * g + i] = (uint8_t)(v >> (8 * i));
    }
  }
}

/* y = W x in double over the f32-dequantized GGUF rows (n_rows rows of k / 256 blocks), as the
 * reference's GEMV tests form their reference (tests/test_q4k_gemv.hip:80-90). */
void oracle_q4k_gemv_f64(const uint8_t* blocks, const float* x, uint32_t n_rows, uint32_t k,
                         double* y) {
  float* w = (float*)malloc(sizeof(float) * k);
  for (uint32_t r = 0; r < n_rows; ++r) {
    oracle_q4k_dequant(blocks + (size_t)r * (k / 256) * 144, k / 256, w, NULL);
    double acc = 0;
    for (uint32_t i = 0; i < k; ++i) acc += (double)w[i] * (double)x[i];
    y[r] = acc;
  }
  free(w);
}

/* Q6_K (attn_v). GGUF block (210 bytes): ql[128], qh[64], int8 scales[16], f16 d;
 * element e: q = (ql[64 (e/128) + e%64] >> 4 ((e%128)/64) & 15) | (qh[32 (e/128) + e%32] >>
 * 2 ((e%128)/32) & 3) << 4, y = (d sc[e/16]) (q - 32) in f32 (src/dequant.cpp:63-75). */
void oracle_q6k_dequant(const uint8_t* blocks, size_t n_blocks, float* out) {
  for (size_t b = 0; b < n_blocks; ++b) {
    const uint8_t* ql = blocks + b * 210;
    const uint8_t* qh = ql + 128;
    const int8_t* sc = (const int8_t*)(ql + 192);
    const float d = f16_at(ql + 208);
    for (int e = 0; e < 256; ++e) {
      const int h = e / 128, r = e % 128;
      const int lo = (ql[h * 64 + r % 64] >> (4 * (r / 64))) & 15;
      const int hi = (qh[h * 32 + r % 32] >> (2 * (r / 32))) & 3;
      const float ds = d * (float)sc[e / 16];
      out[b * 256 + e] = ds * (float)((lo | hi << 4) - 32);
    }
  }
}

/* GGUF rows -> r1 rows (src/repack.cpp:53-74): per row [ql nb x 128][qh nb x 64][scales nb x 16]
 * [d nb x 2], zero-padded to a multiple of 16 bytes. */
void oracle_q6k_repack_r1(const uint8_t* src, uint32_t n_rows, uint32_t k, uint8_t* dst) {
  const size_t nb = k / 256, src_row = nb * 210, dst_row = (nb * 210 + 15) / 16 * 16;
  for (uint32_t r = 0; r < n_rows; ++r) {
    uint8_t* o = dst + r * dst_row;
    memset(o, 0, dst_row);
    for (size_t b = 0; b < nb; ++b) {
      const uint8_t* blk = src + r * src_row + b * 210;
      memcpy(o + b * 128, blk, 128);
      memcpy(o + nb * 128 + b * 64, blk + 128, 64);
      memcpy(o + nb * 192 + b * 16, blk + 192, 16);
      memcpy(o + nb * 208 + b * 2, blk + 208, 2);
    }
  }
}

void oracle_q6k_gemv_f64(const uint8_t* blocks, const float* x, uint32_t n_rows, uint32_t k,
                         double* y) {
  float* w = (float*)malloc(sizeof(float) * k);
  for (uint32_t r = 0; r < n_rows; ++r) {
    oracle_q6k_dequant(blocks + (size_t)r * (k / 256) * 210, k / 256, w);
    double acc = 0;
    for (uint32_t i = 0; i < k; ++i) acc += (double)w[i] * (double)x[i];
    y[r] = acc;
  }
  free(w);
}
