/*
 * catena_oracle.c -- CPU restatement of catena-lang's generated arithmetic
 * for the matmul contraction and the softmax-based decode attention.
 *
 * TEST INFRASTRUCTURE ONLY (see catena_oracle.h).  It is the checker for the
 * HIP kernels and the timed CPU baseline; the product never calls it.
 *
 * Every floating-point statement below is one IEEE binary32 operation in the
 * order the reference's renderer emits it; the file must be compiled with
 * -ffp-contract=off -fno-fast-math (oracle/Makefile) exactly like the
 * reference's generated module (catena-lang/src/runtime/artifact.rs:59-71).
 */
#include "catena_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* catena_u32_bitcast_f32 / catena_f32_bitcast_u32,
 * catena-lang/src/codegen/prelude.rs:64-80 */
uint32_t or_f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

float or_bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

/* f32.round-to-u32 renders as `(uint32_t)nearbyintf(x)`
 * (catena-lang/src/codegen/gpu.rs:642-655).  The C cast is undefined outside
 * [0, 2^32); on the device it is v_cvt_u32_f32, which maps NaN and negatives
 * to 0 and saturates at 0xFFFFFFFF.  That device behaviour is the one this
 * build defines (the exp~ producers run inside device kernels). */
uint32_t or_round_to_u32(float x) {
  float r = nearbyintf(x);
  if (r != r) return 0u;
  if (r <= 0.0f) return 0u;
  if (r >= 4294967296.0f) return 0xFFFFFFFFu;
  return (uint32_t)r;
}

/* math.exp-approx-nonneg, catena-lang/stdlib/math.hex:148-183.
 * One statement per hexpr node, operands in source order. */
float or_exp_approx_nonneg(float x) {
  const float inv_ln2 = or_bits_f32(0x3FB8AA3Bu);
  const float ln2_hi = or_bits_f32(0x3F317200u);
  const float ln2_lo = or_bits_f32(0x35BFBE8Eu);
  const float c0 = or_bits_f32(0x3F7FF8FCu);
  const float c1 = or_bits_f32(0x3F809C7Eu);
  const float c2 = or_bits_f32(0x3EEF1187u);
  const float c3 = or_bits_f32(0x3E738A8Bu);

  float scaled = x * inv_ln2;
  uint32_t k_u32 = or_round_to_u32(scaled);
  float k_f32 = (float)k_u32; /* u32.to-f32 */
  float k_ln2_hi = k_f32 * ln2_hi;
  float k_ln2_lo = k_f32 * ln2_lo;
  float r1 = x - k_ln2_hi;
  float xr = r1 - k_ln2_lo;
  float xr_c3 = xr * c3;
  float p2 = c2 + xr_c3;
  float xr_p2 = xr * p2;
  float p1 = c1 + xr_p2;
  float xr_p1 = xr * p1;
  float poly = c0 + xr_p1;
  uint32_t biased = k_u32 + 0x7Fu;          /* u32.add, wraps */
  uint32_t pow2_bits = biased * 0x00800000u; /* u32.mul, wraps */
  float pow2k = or_bits_f32(pow2_bits);
  return poly * pow2k;
}

/* math.exp-approx, catena-lang/stdlib/math.hex:185-199 */
float or_exp_approx(float x) {
  const float zero = (float)0u;
  const float one = or_bits_f32(0x3F800000u);
  float neg_x = -x;
  int is_negative = x < zero;
  float magnitude = is_negative ? neg_x : x;
  float base = or_exp_approx_nonneg(magnitude);
  float reciprocal = one / base;
  return is_negative ? reciprocal : base;
}

/* or_exp_approx over an array (for sweeps: one call instead of n). */
void or_exp_approx_n(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = or_exp_approx(x[i]);
}

/* f32 -> bf16, round to nearest even.  NaN keeps its sign and top payload
 * bits and is forced quiet.  This conversion has no reference counterpart
 * (catena has no bf16, catena-lang/src/codegen/lower_types.rs:13-22); it is
 * the output rounding this build defines for the bf16 GEMM. */
uint16_t or_f32_to_bf16(float x) {
  uint32_t u = or_f32_bits(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7FFFu + lsb;
  return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t h) { return or_bits_f32(((uint32_t)h) << 16); }

/* sum-f32 via reducec with f32.add-env (catena-lang/stdlib/sum.hex:7-14,
 * fold loop catena-lang/src/codegen/ops/reducec.rs:73-130): acc starts at
 * bitcast(0) = +0.0 and `acc = acc + x_i` in ascending i. */
float or_fold_sum_f32(const float *x, uint64_t n) {
  float acc = or_bits_f32(0u);
  for (uint64_t i = 0; i < n; ++i) {
    float next = acc + x[i];
    acc = next;
  }
  return acc;
}

/* max-f32 via f32.max-env (catena-lang/stdlib/sum.hex:73-84): acc starts at
 * bitcast(0xFF800000) = -inf; keep acc when acc >= x. */
float or_fold_max_f32(const float *x, uint64_t n) {
  float acc = or_bits_f32(0xFF800000u);
  for (uint64_t i = 0; i < n; ++i) {
    int keep = acc >= x[i];
    acc = keep ? acc : x[i];
  }
  return acc;
}

/* ---------------------------------------------------------------------- */
/* thread fan-out over an index range                                      */

typedef void (*or_range_fn)(void *ctx, uint64_t lo, uint64_t hi);

typedef struct {
  or_range_fn fn;
  void *ctx;
  uint64_t lo, hi;
} or_job;

static void *or_job_main(void *p) {
  or_job *j = (or_job *)p;
  j->fn(j->ctx, j->lo, j->hi);
  return NULL;
}

static void or_parallel(or_range_fn fn, void *ctx, uint64_t count, int threads) {
  if (threads <= 1 || count < 2) {
    fn(ctx, 0, count);
    return;
  }
  if ((uint64_t)threads > count) threads = (int)count;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  or_job *jobs = (or_job *)malloc(sizeof(or_job) * (size_t)threads);
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].lo = count * (uint64_t)t / (uint64_t)threads;
    jobs[t].hi = count * (uint64_t)(t + 1) / (uint64_t)threads;
    pthread_create(&tid[t], NULL, or_job_main, &jobs[t]);
  }
  for (int t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}

/* ---------------------------------------------------------------------- */
/* f32.matmul.row-major.materialize                                        */
/*
 * For every flat output index (materializec, catena-lang/src/codegen/ops/
 * materializec.rs:36-82): i = flat / m, j = flat % m (row_major.rs:30-68);
 * cell-dot (catena-lang/stdlib/matrix.hex:236-256) folds k ascending from
 * +0.0 with acc = acc + (A[i*k_len+k] * B[k*m+j]) (matrix.hex:210-233,
 * row_major.rs:9-28).  The loop below walks a whole output row at once with
 * j innermost; each cell still sees its own k-ascending chain, so the
 * result is bitwise the per-cell order.
 */
typedef struct {
  const float *a, *b;
  float *c;
  uint64_t m, k;
} or_mm_f32_ctx;

static void or_mm_f32_rows(void *p, uint64_t lo, uint64_t hi) {
  or_mm_f32_ctx *x = (or_mm_f32_ctx *)p;
  for (uint64_t i = lo; i < hi; ++i) {
    float *crow = x->c + i * x->m;
    for (uint64_t j = 0; j < x->m; ++j) crow[j] = or_bits_f32(0u);
    for (uint64_t kk = 0; kk < x->k; ++kk) {
      const float aik = x->a[i * x->k + kk];
      const float *brow = x->b + kk * x->m;
      for (uint64_t j = 0; j < x->m; ++j) {
        float v = aik * brow[j];
        crow[j] = crow[j] + v;
      }
    }
  }
}

void or_matmul_f32_seq(const float *a, const float *b, float *c, uint64_t n,
                       uint64_t m, uint64_t k, int threads) {
  or_mm_f32_ctx x = {a, b, c, m, k};
  or_parallel(or_mm_f32_rows, &x, n, threads);
}

/* bf16 GEMM: the same fold on exactly widened inputs, then RNE to bf16. */
typedef struct {
  const uint16_t *a, *b;
  float *c32;
  uint16_t *c16;
  uint64_t n, m, k;
  const uint64_t *rows;
} or_mm_bf16_ctx;

static void or_mm_bf16_rows(void *p, uint64_t lo, uint64_t hi) {
  or_mm_bf16_ctx *x = (or_mm_bf16_ctx *)p;
  float *bw = (float *)malloc(sizeof(float) * x->m);
  float *acc = (float *)malloc(sizeof(float) * x->m);
  for (uint64_t idx = lo; idx < hi; ++idx) {
    uint64_t i = x->rows ? x->rows[idx] : idx;
    for (uint64_t j = 0; j < x->m; ++j) acc[j] = or_bits_f32(0u);
    for (uint64_t kk = 0; kk < x->k; ++kk) {
      const float aik = or_bf16_to_f32(x->a[i * x->k + kk]);
      const uint16_t *brow = x->b + kk * x->m;
      for (uint64_t j = 0; j < x->m; ++j) bw[j] = or_bf16_to_f32(brow[j]);
      for (uint64_t j = 0; j < x->m; ++j) {
        float v = aik * bw[j];
        acc[j] = acc[j] + v;
      }
    }
    if (x->c32) memcpy(x->c32 + idx * x->m, acc, sizeof(float) * x->m);
    if (x->c16)
      for (uint64_t j = 0; j < x->m; ++j) x->c16[idx * x->m + j] = or_f32_to_bf16(acc[j]);
  }
  free(bw);
  free(acc);
}

void or_matmul_bf16_seq(const uint16_t *a, const uint16_t *b, float *c32,
                        uint16_t *c16, uint64_t n, uint64_t m, uint64_t k,
                        const uint64_t *rows, uint64_t nrows, int threads) {
  or_mm_bf16_ctx x = {a, b, c32, c16, n, m, k, rows};
  or_parallel(or_mm_bf16_rows, &x, rows ? nrows : n, threads);
}

/* ---------------------------------------------------------------------- */
/* nn.softmax, catena-lang/stdlib/nn.hex:93-122:
 *   max   = reducec(-inf, f32.max-env, x)
 *   denom = reducec(+0,  f32.add-env, exp~(x_i - max))   (nn.hex:59-72)
 *   out_i = exp~(x_i - max) / denom                       (nn.hex:75-90) */
void or_softmax_f32(const float *x, float *y, uint64_t n) {
  float mx = or_fold_max_f32(x, n);
  float den = or_bits_f32(0u);
  for (uint64_t i = 0; i < n; ++i) {
    float shifted = x[i] - mx;
    float e = or_exp_approx(shifted);
    den = den + e;
  }
  for (uint64_t i = 0; i < n; ++i) {
    float shifted = x[i] - mx;
    float e = or_exp_approx(shifted);
    y[i] = e / den;
  }
}

/* ---------------------------------------------------------------------- */
/* Decode attention for one query token per (batch, head).  There is no
 * reference function; it is composed from the reference's pieces:
 *   s_t   = cell-dot over d ascending (matrix.hex:236-256) of q_d * k_{t,d},
 *           then one f32.mul by scale;
 *   p     = nn.softmax(s) exactly as or_softmax_f32 (nn.hex:93-122);
 *   o_d   = cell-dot over t ascending of p_t * v_{t,d}.
 * bf16 inputs are widened exactly.  A head with length 0 yields o = +0. */
typedef struct {
  const uint16_t *q, *k, *v;
  const uint32_t *lens;
  float *o;
  uint32_t H, L, D;
  float scale;
  const uint32_t *bh_list;
} or_attn_ctx;

static void or_attn_heads(void *p, uint64_t lo, uint64_t hi) {
  or_attn_ctx *x = (or_attn_ctx *)p;
  const uint64_t L = x->L, D = x->D;
  float *s = (float *)malloc(sizeof(float) * (L ? L : 1));
  float *qf = (float *)malloc(sizeof(float) * D);
  float *acc = (float *)malloc(sizeof(float) * D);
  for (uint64_t idx = lo; idx < hi; ++idx) {
    uint64_t bh = x->bh_list ? x->bh_list[idx] : idx;
    uint64_t b = bh / x->H;
    uint64_t len = x->lens[b];
    const uint16_t *kb = x->k + bh * L * D;
    const uint16_t *vb = x->v + bh * L * D;
    for (uint64_t d = 0; d < D; ++d) qf[d] = or_bf16_to_f32(x->q[bh * D + d]);
    for (uint64_t t = 0; t < len; ++t) {
      float a = or_bits_f32(0u);
      for (uint64_t d = 0; d < D; ++d) {
        float prod = qf[d] * or_bf16_to_f32(kb[t * D + d]);
        a = a + prod;
      }
      s[t] = a * x->scale;
    }
    if (len > 0) or_softmax_f32(s, s, len);
    for (uint64_t d = 0; d < D; ++d) acc[d] = or_bits_f32(0u);
    for (uint64_t t = 0; t < len; ++t) {
      const float pt = s[t];
      for (uint64_t d = 0; d < D; ++d) {
        float prod = pt * or_bf16_to_f32(vb[t * D + d]);
        acc[d] = acc[d] + prod;
      }
    }
    memcpy(x->o + (x->bh_list ? idx : bh) * D, acc, sizeof(float) * D);
  }
  free(s);
  free(qf);
  free(acc);
}

void or_attn_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    const uint32_t *lens, float *o, uint32_t B, uint32_t H,
                    uint32_t L, uint32_t D, float scale,
                    const uint32_t *bh_list, uint32_t nbh, int threads) {
  or_attn_ctx x = {q, k, v, lens, o, H, L, D, scale, bh_list};
  uint64_t count = bh_list ? nbh : (uint64_t)B * H;
  or_parallel(or_attn_heads, &x, count, threads);
}
