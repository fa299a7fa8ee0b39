/*
 * catena_oracle.h -- CPU restatement of the arithmetic that catena-lang's
 * generated code performs on the GEMM-contraction and softmax/attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product path may link or call
 * this library; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker / the timed CPU baseline.
 *
 * Build contract (mirrors catena-lang/src/runtime/artifact.rs:59-71):
 * compiled with -O2 -ffp-contract=off -fno-fast-math so every `*` and `+`
 * is a separately rounded IEEE binary32 operation and nothing is
 * reassociated or contracted into an FMA.
 *
 * Pinning status (each function is checked in tests/test_oracle.py):
 *   or_matmul_f32_seq     pinned: reference known answers
 *                         (tests/cases/matrix.rs:5-82), numpy float32
 *                         sequential fold (bitwise), float64 error bound.
 *   or_exp_approx         pinned: reference tolerance test
 *                         (tests/runtime.rs:742-761), closed-form specials
 *                         (exp~(0)=c0, k=128 -> inf, k=129 -> -0 bits),
 *                         libm relative-error bound over a dense sweep, and
 *                         bitwise over all 2^32 inputs against an independent
 *                         numpy float32 transcription of math.hex:148-199
 *                         (tests/test_oracle_exp_sweep.py).
 *   or_softmax_f32        pinned: reference test (tests/runtime.rs:971-1009),
 *                         sum-to-one, permutation/shift invariants.
 *   or_fold_*_f32         pinned: reference known answers
 *                         (tests/cases/reducec.rs:50-90).
 *   or_f32_to_bf16        pinned: torch's RNE float->bfloat16 conversion.
 *   or_matmul_bf16_*      pinned: bitwise or_matmul_f32_seq on exactly
 *                         widened inputs (ragged shapes), float64 error
 *                         bound, exact integer cases.
 *   or_attn_decode        pinned: float64 attention within the softmax
 *                         tolerance, brute-force composition of the pinned
 *                         pieces on tiny shapes, uniform-V / one-hot cases.
 *   or_sqrt_newton        pinned: closed forms (1, 4, 0, negatives), libm on
 *                         the converging range, the reference's divergence
 *                         for large inputs (guess0 = x).
 *   or_sigmoid/or_silu    pinned: closed form at 0, libm within exp~'s error.
 *   or_sin/cos_full       pinned: libm within the Taylor remainder bound,
 *                         exact 0/1 at 0, odd/even symmetry.
 *   or_rmsnorm_f32        pinned: reference test (tests/runtime.rs:1011-1044).
 *   or_argmax_f32         pinned: reference cases (tests/runtime.rs:1176-1197).
 *   or_rope_f32           pinned: identity at pos 0, norm preservation,
 *                         float64 rotation with libm cos/sin.
 */
#ifndef CATENA_ORACLE_H
#define CATENA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* scalar pieces */
uint32_t or_f32_bits(float x);
float or_bits_f32(uint32_t b);
uint32_t or_round_to_u32(float x);
float or_exp_approx_nonneg(float x);
float or_exp_approx(float x);
void or_exp_approx_n(const float *x, float *y, uint64_t n);
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t h);

/* folds (sum.hex) */
float or_fold_sum_f32(const float *x, uint64_t n);
float or_fold_max_f32(const float *x, uint64_t n);

/* f32.matmul.row-major.materialize: C[n x m] = A[n x k] * B[k x m] */
void or_matmul_f32_seq(const float *a, const float *b, float *c,
                       uint64_t n, uint64_t m, uint64_t k, int threads);

/* bf16 GEMM defined on the same fold: inputs widened exactly to f32.
 * rows != NULL restricts the computation to the listed output rows
 * (row r of the result goes to c32 + idx*m). c16 may be NULL. */
void or_matmul_bf16_seq(const uint16_t *a, const uint16_t *b, float *c32,
                        uint16_t *c16, uint64_t n, uint64_t m, uint64_t k,
                        const uint64_t *rows, uint64_t nrows, int threads);

/* nn.softmax over one f32 vector (n >= 1) */
void or_softmax_f32(const float *x, float *y, uint64_t n);

/* decode attention: q[B,H,D], k/v[B,H,L,D] bf16, lens[B], o[B,H,D] f32.
 * bh_list != NULL restricts to the listed (b*H+h) heads; head idx of the
 * list writes o + idx*D. */
void or_attn_decode(const uint16_t *q, const uint16_t *k, const uint16_t *v,
                    const uint32_t *lens, float *o, uint32_t B, uint32_t H,
                    uint32_t L, uint32_t D, float scale,
                    const uint32_t *bh_list, uint32_t nbh, int threads);

/* ---- decoder-block pieces (catena_oracle_block.c) ---- */
float or_sqrt_newton(float x);   /* math.sqrt */
float or_sigmoid(float x);       /* nn.sigmoid */
float or_silu(float x);          /* nn.silu */
float or_sin_approx(float x);    /* math.sin-approx */
float or_cos_approx(float x);    /* math.cos-approx */
float or_sin_full(float x);      /* math.sin-approx-full */
float or_cos_full(float x);      /* this build's full-range cosine */
/* ops 0..6: exp-approx, sqrt, sigmoid, silu, sin-approx, cos-approx, sin-approx-full */
void or_map_f32(int op, const float *x, float *y, uint64_t n);
void or_rmsnorm_f32(const float *x, float *y, uint64_t n);   /* nn.rmsnorm */
uint64_t or_argmax_f32(const float *x, uint64_t n);           /* tensor.argmax-f32 */
void or_rope_inv_freq(float *inv_freq, uint32_t d, double base);
void or_rope_f32(float *x, uint32_t pos, const float *inv_freq, uint32_t d);
/* whole-activation forms of the decoder stages (row by row, same bits) */
void or_silu_mul_rows(const float *gu, uint16_t *out, uint64_t rows, uint32_t ffn,
                      uint32_t group);
void or_rope_qkv_rows(const float *qkv, const float *inv_freq, const uint32_t *pos,
                      uint16_t *q, uint16_t *k, uint16_t *v, uint64_t rows, uint32_t heads,
                      uint32_t d);
void or_rmsnorm_rows(const float *x, float *y, uint64_t rows, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
