/*
 * catena_oracle_block.c -- CPU restatement of the stdlib pieces a
 * Llama-style decoder block is built from (nn.rmsnorm, math.sqrt, nn.silu,
 * math.sin-approx-full, tensor.argmax-f32) plus the RoPE rotation this build
 * defines on top of them.
 *
 * TEST INFRASTRUCTURE ONLY (see catena_oracle.h).  Same compile contract
 * (-ffp-contract=off -fno-fast-math): one IEEE binary32 operation per hexpr
 * node, operands in source order.
 */
#include <math.h>
#include <string.h>

#include "catena_oracle.h"

/* math.sqrt, catena-lang/stdlib/math.hex:235-272: six Newton steps from
 * guess0 = (x < 1) ? 1 : x; non-positive inputs give +0. */
float or_sqrt_newton(float x) {
  const float zero = (float)0u;
  const float one = or_bits_f32(0x3F800000u);
  const float half = or_bits_f32(0x3F000000u);
  int lt_one = x < one;
  float g = lt_one ? one : x;
  for (int it = 0; it < 6; ++it) {
    float ratio = x / g;
    float sum = g + ratio;
    g = sum * half;
  }
  int is_nonpositive = x <= zero;
  return is_nonpositive ? zero : g;
}

/* nn.sigmoid, catena-lang/stdlib/nn.hex:1-12: 1 / (1 + exp~(-x)) */
float or_sigmoid(float x) {
  const float one = 1.0f; /* f32.one renders as `= 1.0` */
  float neg_x = -x;
  float e = or_exp_approx(neg_x);
  float den = one + e;
  return one / den;
}

/* nn.silu, catena-lang/stdlib/nn.hex:14-21: x * sigmoid(x) */
float or_silu(float x) {
  float gate = or_sigmoid(x);
  return x * gate;
}

/* math.sin-approx, catena-lang/stdlib/math.hex:1-24 */
float or_sin_approx(float x) {
  float x2 = x * x;
  float x3 = x2 * x;
  float x5 = x3 * x2;
  float x7 = x5 * x2;
  const float f3 = (float)6u, f5 = (float)120u, f7 = (float)5040u;
  float a = x3 / f3;
  float b = x5 / f5;
  float c = x7 / f7;
  float p1 = x - a;
  float p2 = p1 + b;
  return p2 - c;
}

/* math.cos-approx, catena-lang/stdlib/math.hex:26-47 */
float or_cos_approx(float x) {
  float x2 = x * x;
  float x4 = x2 * x2;
  float x6 = x4 * x2;
  const float f2 = (float)2u, f4 = (float)24u, f6 = (float)720u, one = (float)1u;
  float a = x2 / f2;
  float b = x4 / f4;
  float c = x6 / f6;
  float p1 = one - a;
  float p2 = p1 + b;
  return p2 - c;
}

/* Cody-Waite quadrant evaluation shared by sin and cos:
 * catena-lang/stdlib/math.hex:52-88 with the quadrant offset `shift`
 * (0 for math.sin-approx-full-nonneg; 1 for the cosine defined below). */
static float or_quadrant_eval(float x, uint32_t shift) {
  const float inv_pio2 = or_bits_f32(0x3F22F983u);
  const float pio2_hi = or_bits_f32(0x3FC90FDAu);
  const float pio2_lo = or_bits_f32(0x33A22168u);
  float scaled = x * inv_pio2;
  uint32_t n_u32 = or_round_to_u32(scaled);
  float n_f = (float)n_u32;
  float n_hi = n_f * pio2_hi;
  float n_lo = n_f * pio2_lo;
  float r1 = x - n_hi;
  float r = r1 - n_lo;
  float sin_r = or_sin_approx(r);
  float cos_r = or_cos_approx(r);
  float neg_sin = -sin_r;
  float neg_cos = -cos_r;
  uint32_t quadrant = (n_u32 + shift) & 3u;
  int is_q0 = quadrant == 0u, is_q1 = quadrant == 1u, is_q2 = quadrant == 2u;
  float q23 = is_q2 ? neg_sin : neg_cos;
  float q123 = is_q1 ? cos_r : q23;
  return is_q0 ? sin_r : q123;
}

/* math.sin-approx-full, catena-lang/stdlib/math.hex:90-103: odd extension */
float or_sin_full(float x) {
  const float zero = (float)0u;
  float neg_x = -x;
  int is_negative = x < zero;
  float magnitude = is_negative ? neg_x : x;
  float base = or_quadrant_eval(magnitude, 0u);
  float negated = -base;
  return is_negative ? negated : base;
}

/* Full-range cosine, defined by this build (the stdlib has only the Taylor
 * math.cos-approx): cos(x) = sin(|x| + pi/2) evaluated with the same
 * reduction as math.sin-approx-full-nonneg and the quadrant advanced by one,
 * so no rounding is added by forming |x| + pi/2. */
float or_cos_full(float x) {
  const float zero = (float)0u;
  float neg_x = -x;
  int is_negative = x < zero;
  float magnitude = is_negative ? neg_x : x;
  return or_quadrant_eval(magnitude, 1u);
}

/* nn.rmsnorm, catena-lang/stdlib/nn.hex:154-182 (no gain: the Llama gain
 * of ones is the identity). */
/* The scalar programs over an array, selected by op (the numbering of
 * catena_map_op_t in the library's header): 0 exp-approx, 1 sqrt,
 * 2 sigmoid, 3 silu, 4 sin-approx, 5 cos-approx, 6 sin-approx-full. */
void or_map_f32(int op, const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    const float v = x[i];
    switch (op) {
      case 0: y[i] = or_exp_approx(v); break;
      case 1: y[i] = or_sqrt_newton(v); break;
      case 2: y[i] = or_sigmoid(v); break;
      case 3: y[i] = or_silu(v); break;
      case 4: y[i] = or_sin_approx(v); break;
      case 5: y[i] = or_cos_approx(v); break;
      default: y[i] = or_sin_full(v); break;
    }
  }
}

void or_rmsnorm_f32(const float *x, float *y, uint64_t n) {
  float sum_sq = or_bits_f32(0u);
  for (uint64_t i = 0; i < n; ++i) {
    float sq = x[i] * x[i];
    sum_sq = sum_sq + sq;
  }
  float len_f = (float)n; /* u64.to-f32 */
  float mean_sq = sum_sq / len_f;
  const float eps = or_bits_f32(0x3727C5ACu);
  float t = mean_sq + eps;
  float rms = or_sqrt_newton(t);
  for (uint64_t i = 0; i < n; ++i) y[i] = x[i] / rms;
}

/* tensor.argmax-f32, catena-lang/stdlib/tensor.hex:204-227: acc starts at
 * (0, x[0]); for every i ascending keep acc when acc.max >= x[i]. */
uint64_t or_argmax_f32(const float *x, uint64_t n) {
  uint64_t pos = 0;
  float mx = x[0];
  for (uint64_t i = 0; i < n; ++i) {
    int keep = mx >= x[i];
    pos = keep ? pos : i;
    mx = keep ? mx : x[i];
  }
  return pos;
}

/* RoPE inverse frequencies (this build's definition): inv_freq[i] =
 * (float)(1 / base^(2i/d)) computed in double precision, i < d/2. */
void or_rope_inv_freq(float *inv_freq, uint32_t d, double base) {
  for (uint32_t i = 0; i < d / 2; ++i) inv_freq[i] = (float)(1.0 / pow(base, (2.0 * i) / d));
}

/* Rotate one head vector of length d (half-split pairs x[i], x[i + d/2]) at
 * position pos: theta = (float)pos * inv_freq[i]; y1 = x1 c - x2 s;
 * y2 = x2 c + x1 s, each product and sum separately rounded. */
void or_rope_f32(float *x, uint32_t pos, const float *inv_freq, uint32_t d) {
  const uint32_t h = d / 2;
  const float pf = (float)pos;
  for (uint32_t i = 0; i < h; ++i) {
    float theta = pf * inv_freq[i];
    float c = or_cos_full(theta);
    float s = or_sin_full(theta);
    float x1 = x[i], x2 = x[i + h];
    float t1 = x1 * c, t2 = x2 * s;
    float t3 = x2 * c, t4 = x1 * s;
    x[i] = t1 - t2;
    x[i + h] = t3 + t4;
  }
}

/* Whole-activation forms of the two elementwise decoder stages, row by row
 * through the functions above (checkers for full-size activations).
 *
 * SwiGLU gate: out[r][i] = bf16(nn.silu(gate) * up) with one f32 rounding of
 * the product; group = 0: gate = gu[r][i], up = gu[r][ffn + i]; group = G:
 * gate and up interleaved in blocks of G columns (gate i at G-block i/G,
 * offset i%G; up G columns after it). */
void or_silu_mul_rows(const float *gu, uint16_t *out, uint64_t rows, uint32_t ffn,
                      uint32_t group) {
  for (uint64_t r = 0; r < rows; ++r) {
    const float *row = gu + r * 2ull * ffn;
    for (uint32_t i = 0; i < ffn; ++i) {
      uint64_t gi, ui;
      if (group == 0) {
        gi = i;
        ui = (uint64_t)ffn + i;
      } else {
        const uint64_t blk = i / group, j = i % group;
        gi = blk * 2ull * group + j;
        ui = gi + group;
      }
      const float s = or_silu(row[gi]);
      const float p = s * row[ui];
      out[r * ffn + i] = or_f32_to_bf16(p);
    }
  }
}

/* RoPE + split of a fused projection row qkv[r][3 * heads * d] (q heads |
 * k heads | v heads) at position pos[r]: q and k heads rotated by
 * or_rope_f32, v copied; all three rounded to bf16.  q[r][heads * d],
 * k / v[r][heads][d]. */
void or_rope_qkv_rows(const float *qkv, const float *inv_freq, const uint32_t *pos,
                      uint16_t *q, uint16_t *k, uint16_t *v, uint64_t rows, uint32_t heads,
                      uint32_t d) {
  float buf[1024];
  const uint64_t hd = (uint64_t)heads * d;
  if (d > 1024) return;
  for (uint64_t r = 0; r < rows; ++r) {
    const float *row = qkv + r * 3 * hd;
    for (uint32_t h = 0; h < heads; ++h) {
      memcpy(buf, row + (uint64_t)h * d, d * sizeof(float));
      or_rope_f32(buf, pos[r], inv_freq, d);
      for (uint32_t i = 0; i < d; ++i) q[r * hd + (uint64_t)h * d + i] = or_f32_to_bf16(buf[i]);
      memcpy(buf, row + hd + (uint64_t)h * d, d * sizeof(float));
      or_rope_f32(buf, pos[r], inv_freq, d);
      for (uint32_t i = 0; i < d; ++i) k[r * hd + (uint64_t)h * d + i] = or_f32_to_bf16(buf[i]);
      for (uint32_t i = 0; i < d; ++i)
        v[r * hd + (uint64_t)h * d + i] = or_f32_to_bf16(row[2 * hd + (uint64_t)h * d + i]);
    }
  }
}

/* nn.rmsnorm of each of `rows` contiguous rows of length n. */
void or_rmsnorm_rows(const float *x, float *y, uint64_t rows, uint64_t n) {
  for (uint64_t r = 0; r < rows; ++r) or_rmsnorm_f32(x + r * n, y + r * n, n);
}
