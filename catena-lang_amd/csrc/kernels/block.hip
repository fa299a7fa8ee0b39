// Decoder-block kernels around the two hot contractions: embedding gather,
// RMSNorm (with the residual add in front), RoPE + KV-cache append, the
// SwiGLU gate and greedy argmax.  Every output is bitwise equal to the
// sequential restatement of the reference's stdlib op it mirrors:
//   nn.rmsnorm          catena-lang/stdlib/nn.hex:154-182 (math.sqrt,
//                       catena-lang/stdlib/math.hex:235-272)
//   nn.silu             catena-lang/stdlib/nn.hex:1-21
//   math.sin-approx-full catena-lang/stdlib/math.hex:52-103 (RoPE's sin; its
//                       cos is the same reduction with the quadrant advanced)
//   tensor.argmax-f32   catena-lang/stdlib/tensor.hex:171-227
// Serial folds stay serial (one lane over LDS, ascending index); everything
// elementwise is one IEEE op per reference node (no contraction: the build
// passes -ffp-contract=off).
#include "common.h"

namespace {
constexpr uint32_t kNaNBits = 0x7FC00000u;

CATENA_DEV int block_max_i32(int v, int* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = red[w] > r ? red[w] : r;
  __syncthreads();
  return r;
}

CATENA_DEV FirstMax block_first_max(FirstMax a, float* red_v, uint32_t* red_u) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    FirstMax b;
    b.v = __shfl_xor(a.v, off, 64);
    b.i = (uint32_t)__shfl_xor((int)a.i, off, 64);
    a = first_max_combine(a, b);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red_v[wave] = a.v;
    red_u[wave] = a.i;
  }
  __syncthreads();
  FirstMax r{red_v[0], red_u[0]};
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = first_max_combine(r, FirstMax{red_v[w], red_u[w]});
  __syncthreads();
  return r;
}
}  // namespace

// x[r][:] = widen(table[tokens[r]][:]).  A token >= V yields a row of NaN
// (no read outside the table).  grid = (ceil(d / 2048), R), block = 256,
// 8 elements per thread; requires d % 8 == 0.
extern "C" __global__ __launch_bounds__(256) void catena_embed_rows_bf16(
    const uint32_t* __restrict__ tokens, const uint16_t* __restrict__ table,
    float* __restrict__ x, uint32_t V, uint32_t d) {
  const uint32_t r = blockIdx.y;
  const uint32_t c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= d) return;
  const uint32_t tok = tokens[r];
  f32x4_t lo, hi;
  if (tok < V) {
    const u32x4_t w = *reinterpret_cast<const u32x4_t*>(table + (uint64_t)tok * d + c);
    lo = f32x4_t{bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1])};
    hi = f32x4_t{bf16lo(w[2]), bf16hi(w[2]), bf16lo(w[3]), bf16hi(w[3])};
  } else {
    const float nan = __uint_as_float(kNaNBits);
    lo = hi = f32x4_t{nan, nan, nan, nan};
  }
  float* dst = x + (uint64_t)r * d + c;
  *reinterpret_cast<f32x4_t*>(dst) = lo;
  *reinterpret_cast<f32x4_t*>(dst + 4) = hi;
}

// One workgroup per output row.  h = x[src] (+ resid[src] when resid is
// given: one f32 add per element); then nn.rmsnorm of h:
//   sum_sq = fold_{i asc} from +0 of h_i * h_i   (one wave,
//            serial_sum_wave_long)
//   rms    = math.sqrt(sum_sq / (f32)n + 0x3727C5AC)
//   y_i    = h_i / rms
// src = row_index ? row_index[row] : row.  Outputs (each optional): h_out
// (f32), y_f32, y_bf16 (RNE).  LDS: 2 * round_up(n, 4) floats.  Rows are
// moved with 16-byte accesses when n % 4 == 0 (pointers 16-byte aligned),
// element by element otherwise.
namespace {
CATENA_DEV void rms_finish_row(const float* hs, uint32_t n, uint64_t row, float rms,
                               float* __restrict__ y_f32, uint16_t* __restrict__ y_bf16) {
  if (n % 4 == 0) {
    for (uint32_t i = threadIdx.x; i < n / 4; i += blockDim.x) {
      const f32x4_t h = reinterpret_cast<const f32x4_t*>(hs)[i];
      f32x4_t y;
#pragma unroll
      for (int j = 0; j < 4; ++j) y[j] = h[j] / rms;
      if (y_f32) reinterpret_cast<f32x4_t*>(y_f32 + row * n)[i] = y;
      if (y_bf16) {
        uint2 p;
        p.x = pack_bf16x2(y[0], y[1]);
        p.y = pack_bf16x2(y[2], y[3]);
        reinterpret_cast<uint2*>(y_bf16 + row * n)[i] = p;
      }
    }
  } else {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
      const float y = hs[i] / rms;
      if (y_f32) y_f32[row * n + i] = y;
      if (y_bf16) y_bf16[row * n + i] = (uint16_t)f32_to_bf16_bits(y);
    }
  }
}
}  // namespace

// With tokens given, the input row is the embedding gather
// widen(table[tokens[src]]) (a token >= vocab gives NaN) instead of x[src];
// with a table but neither x nor tokens, it is widen(table[src]) (src >=
// vocab gives NaN), which builds the normalized table of every token.
// resid may come as the k-group partials of the decode GEMM that produced it
// (resid_parts > 1, part s at resid + s * resid_stride): resid[src] is then
// ((P0 + P1) + ...) + P(parts-1), the adds that GEMM's own reduction makes.
// resid[src] (the sum) is written to resid_out[src] when resid_out is given.
extern "C" __global__ __launch_bounds__(256) void catena_rmsnorm_rows(
    const float* __restrict__ x, const float* __restrict__ resid,
    const uint32_t* __restrict__ row_index, float* __restrict__ h_out,
    float* __restrict__ y_f32, uint16_t* __restrict__ y_bf16, uint32_t n,
    const uint32_t* __restrict__ tokens, const uint16_t* __restrict__ table, uint32_t vocab,
    uint32_t resid_parts, uint64_t resid_stride, float* __restrict__ resid_out) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const uint32_t n_pad = (n + 3u) & ~3u;
  float* hs = reinterpret_cast<float*>(smem);  // [n_pad]
  float* sq = hs + n_pad;                      // [n_pad]
  __shared__ float rms_s;
  const uint32_t row = blockIdx.x;
  const uint64_t src = row_index ? row_index[row] : row;
  uint32_t tok = 0;
  bool tok_ok = true;
  const bool gather = tokens || (!x && table);
  if (gather) {
    tok = tokens ? tokens[src] : (uint32_t)src;
    tok_ok = tok < vocab;
  }
  const float nan = __uint_as_float(kNaNBits);
  if (n % 4 == 0) {
    const f32x4_t* x4 = reinterpret_cast<const f32x4_t*>(x + src * n);
    const f32x4_t* r4 = resid ? reinterpret_cast<const f32x4_t*>(resid + src * n) : nullptr;
    const uint2* e4 = gather ? reinterpret_cast<const uint2*>(table + (uint64_t)tok * n) : nullptr;
    for (uint32_t i = threadIdx.x; i < n / 4; i += 256) {
      f32x4_t h;
      if (gather) {
        if (tok_ok) {
          const uint2 w = e4[i];
          h = f32x4_t{bf16lo(w.x), bf16hi(w.x), bf16lo(w.y), bf16hi(w.y)};
        } else {
          h = f32x4_t{nan, nan, nan, nan};
        }
      } else {
        h = x4[i];
      }
      if (r4) {
        f32x4_t rr = r4[i];
        if (resid_parts > 1) {
          // every part's load in flight before the adds (up to 8 at once)
          const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(resid + resid_stride + src * n);
          const uint64_t st4 = resid_stride / 4;
          for (uint32_t s0 = 1; s0 < resid_parts; s0 += 8) {
            f32x4_t pp[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
              if (s0 + u < resid_parts) pp[u] = p4[(s0 - 1 + u) * st4 + i];
#pragma unroll
            for (int u = 0; u < 8; ++u)
              if (s0 + u < resid_parts) {
#pragma unroll
                for (int j = 0; j < 4; ++j) rr[j] = rr[j] + pp[u][j];
              }
          }
        }
        if (resid_out) reinterpret_cast<f32x4_t*>(resid_out + src * n)[i] = rr;
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = h[j] + rr[j];
      }
      f32x4_t s;
#pragma unroll
      for (int j = 0; j < 4; ++j) s[j] = h[j] * h[j];
      reinterpret_cast<f32x4_t*>(hs)[i] = h;
      reinterpret_cast<f32x4_t*>(sq)[i] = s;
      if (h_out) reinterpret_cast<f32x4_t*>(h_out + (uint64_t)row * n)[i] = h;
    }
  } else {
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
      float h;
      if (gather)
        h = tok_ok ? bf16_to_f32(table[(uint64_t)tok * n + i]) : nan;
      else
        h = x[src * n + i];
      if (resid) {
        float rr = resid[src * n + i];
        for (uint32_t s0 = 1; s0 < resid_parts; ++s0) rr = rr + resid[s0 * resid_stride + src * n + i];
        if (resid_out) resid_out[src * n + i] = rr;
        h = h + rr;
      }
      hs[i] = h;
      sq[i] = h * h;
      if (h_out) h_out[(uint64_t)row * n + i] = h;
    }
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const float sum_sq = serial_sum_wave_long(sq, n);
    if (threadIdx.x == 0) {
      const float len_f = (float)(uint64_t)n;
      const float mean_sq = sum_sq / len_f;
      const float eps = u32_as_f32(0x3727C5ACu);
      const float t = mean_sq + eps;
      rms_s = sqrt_newton(t);
    }
  }
  __syncthreads();
  rms_finish_row(hs, n, row, rms_s, y_f32, y_bf16);
}

// RoPE on the q and k parts of a fused projection, bf16 q out, and the
// KV-cache append.  qkv[R][3*H*D] f32 with R = B * Tq rows (row b*Tq + tq,
// columns q heads | k heads | v heads); the row's position is
// pos = lens[b] - Tq + tq (lens counts the positions after the append).
// For each head and pair i < D/2 (half-split pairs i, i + D/2):
//   theta = (f32)pos * inv_freq[i];  c = cos_full(theta), s = sin_full(theta)
//   y1 = x1 * c - x2 * s;  y2 = x2 * c + x1 * s   (each op rounded)
// q_out[R][H*D] = bf16(rotated q); kc/vc[B][H][L][D] at pos = bf16(rotated
// k), bf16(v).  Rows whose position falls outside [0, L) write no cache.
// One thread per (row, head, pair); grid = ceil(R*H*D/2 / 256).
extern "C" __global__ __launch_bounds__(256) void catena_rope_qkv_store(
    const float* __restrict__ qkv, const float* __restrict__ inv_freq,
    const uint32_t* __restrict__ lens, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, uint32_t R, uint32_t Tq, uint32_t H, uint32_t D, uint32_t L) {
  const uint32_t half = D / 2;
  const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  const uint64_t per_row = (uint64_t)H * half;
  if (id >= (uint64_t)R * per_row) return;
  const uint32_t r = (uint32_t)(id / per_row);
  const uint32_t rem = (uint32_t)(id % per_row);
  const uint32_t h = rem / half, i = rem % half;
  const uint32_t b = r / Tq, tq = r % Tq;
  const uint32_t len = lens[b];
  const bool pos_ok = len >= Tq && len - Tq + tq < L;
  const uint32_t pos = pos_ok ? len - Tq + tq : 0u;

  const float pf = (float)pos;
  const float theta = pf * inv_freq[i];
  const float c = cos_full(theta);
  const float s = sin_full(theta);
  const uint64_t HD = (uint64_t)H * D;
  const float* src = qkv + (uint64_t)r * 3 * HD + (uint64_t)h * D;
  {
    const float x1 = src[i], x2 = src[i + half];
    const float t1 = x1 * c, t2 = x2 * s, t3 = x2 * c, t4 = x1 * s;
    const float y1 = t1 - t2, y2 = t3 + t4;
    uint16_t* dq = q_out + (uint64_t)r * HD + (uint64_t)h * D;
    dq[i] = (uint16_t)f32_to_bf16_bits(y1);
    dq[i + half] = (uint16_t)f32_to_bf16_bits(y2);
  }
  if (!pos_ok) return;
  const uint64_t cache = (((uint64_t)b * H + h) * L + pos) * D;
  {
    const float x1 = src[HD + i], x2 = src[HD + i + half];
    const float t1 = x1 * c, t2 = x2 * s, t3 = x2 * c, t4 = x1 * s;
    const float y1 = t1 - t2, y2 = t3 + t4;
    kc[cache + i] = (uint16_t)f32_to_bf16_bits(y1);
    kc[cache + i + half] = (uint16_t)f32_to_bf16_bits(y2);
  }
  vc[cache + i] = (uint16_t)f32_to_bf16_bits(src[2 * HD + i]);
  vc[cache + i + half] = (uint16_t)f32_to_bf16_bits(src[2 * HD + i + half]);
}

// The rotation pairs of every position: tab[pos][i] = (cos_full(theta),
// sin_full(theta)) with theta = (f32)pos * inv_freq[i], the values
// catena_rope_qkv_store computes for that position (a table of them gives
// the same bits).  One thread per (pos, i); grid = (ceil(half / 256),
// positions).
extern "C" __global__ __launch_bounds__(256) void catena_rope_table(
    const float* __restrict__ inv_freq, float* __restrict__ tab, uint32_t positions, uint32_t half) {
  const uint32_t pos = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
  if (i >= half) return;
  const uint64_t id = (uint64_t)pos * half + i;
  const float pf = (float)pos;
  const float theta = pf * inv_freq[i];
  tab[2 * id] = cos_full(theta);
  tab[2 * id + 1] = sin_full(theta);
}

// SwiGLU gate: gu[R][2F] f32 -> out[R][F] = bf16(nn.silu(gate) * up).
// group = 0: gate columns [0, F), up columns [F, 2F); group = G: columns
// interleaved in groups of G (gate 0..G-1, up 0..G-1, gate G..2G-1, ...).
// 4 elements per thread; requires F % 4 == 0 and G % 4 == 0.
// grid = (ceil(F / 1024), R).
extern "C" __global__ __launch_bounds__(256) void catena_silu_mul_bf16(
    const float* __restrict__ gu, uint16_t* __restrict__ out, uint32_t F, uint32_t group) {
  const uint32_t r = blockIdx.y;
  const uint32_t c = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (c >= F) return;
  const float* row = gu + (uint64_t)r * 2 * F;
  const uint32_t gcol = group ? (c / group) * 2 * group + c % group : c;
  const uint32_t ucol = gcol + (group ? group : F);
  const f32x4_t g = *reinterpret_cast<const f32x4_t*>(row + gcol);
  const f32x4_t u = *reinterpret_cast<const f32x4_t*>(row + ucol);
  float a[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float act = silu_approx(g[j]);
    a[j] = act * u[j];
  }
  uint2 p;
  p.x = pack_bf16x2(a[0], a[1]);
  p.y = pack_bf16x2(a[2], a[3]);
  *reinterpret_cast<uint2*>(out + (uint64_t)r * F + c) = p;
}

// tensor.argmax-f32 per row: x[R][n] -> idx[R] (u32).  The sequential fold
// keeps (pos, max) while max >= x_i; a NaN therefore replaces the
// accumulator and is itself replaced by the next element, so the result is
// the last NaN when it is the final element, else the first maximum of the
// elements after the last NaN (FirstMax in common.h).  n = 0 writes
// 0xFFFFFFFF (the reference asserts n != 0).
//
// grid = (chunks, R): workgroup c covers [c*chunk, min(n, (c+1)*chunk)) and
// reduces it to (J_c = last NaN index or -1, first max after J_c).  Chunks
// compose in index order: a chunk holding a NaN replaces the state, one
// without merges its first max into it.  The last workgroup of a row (by
// completion ticket) composes the row's chunks in ascending order.
// partials: R x chunks x {J, max bits, index}; tickets[R] start at zero.
extern "C" __global__ __launch_bounds__(256) void catena_argmax_rows_f32(
    const float* __restrict__ x, uint32_t* __restrict__ idx, uint32_t n, uint32_t chunk,
    uint32_t* __restrict__ tickets, uint32_t* __restrict__ partials) {
  __shared__ int red_i[4];
  __shared__ float red_v[4];
  __shared__ uint32_t red_u[4];
  __shared__ uint32_t last_flag;
  const uint32_t row = blockIdx.y;
  const float* xr = x + (uint64_t)row * n;
  if (n == 0) {
    if (threadIdx.x == 0 && blockIdx.x == 0) idx[row] = 0xFFFFFFFFu;
    return;
  }
  const uint32_t beg = blockIdx.x * chunk;
  const uint32_t end = beg + chunk < n ? beg + chunk : n;
  constexpr int PER = 16;  // elements per thread per batch
  int lastnan = -1;
  for (uint32_t b0 = beg; b0 < end; b0 += 256 * PER) {
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t i = b0 + threadIdx.x + 256 * k;
      v[k] = i < end ? xr[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t i = b0 + threadIdx.x + 256 * k;
      if (i < end && v[k] != v[k]) lastnan = (int)i;
    }
  }
  const int J = block_max_i32(lastnan, red_i);
  FirstMax fm{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
  for (uint32_t b0 = beg; b0 < end; b0 += 256 * PER) {
    float v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t i = b0 + threadIdx.x + 256 * k;
      v[k] = i < end ? xr[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const uint32_t i = b0 + threadIdx.x + 256 * k;
      if (i < end && (int)i > J) fm = first_max_combine(fm, FirstMax{v[k], i});
    }
  }
  const FirstMax part = block_first_max(fm, red_v, red_u);
  const uint32_t chunks = gridDim.x;
  if (chunks == 1) {
    if (threadIdx.x == 0) idx[row] = (J == (int)n - 1) ? (uint32_t)J : part.i;
    return;
  }
  uint32_t* pr = partials + 3ull * ((uint64_t)row * chunks);
  if (threadIdx.x == 0) {
    store_coherent(&pr[3 * blockIdx.x + 0], (uint32_t)J);
    store_coherent(&pr[3 * blockIdx.x + 1], __float_as_uint(part.v));
    store_coherent(&pr[3 * blockIdx.x + 2], part.i);
  }
  if (!last_arrival(&tickets[row], chunks, &last_flag)) return;
  if (threadIdx.x != 0) return;
  int sj = -1;
  FirstMax st{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
  for (uint32_t c = 0; c < chunks; ++c) {
    const int jc = (int)load_coherent(&pr[3 * c]);
    const FirstMax fc{__uint_as_float(load_coherent(&pr[3 * c + 1])), load_coherent(&pr[3 * c + 2])};
    if (jc >= 0) {
      sj = jc;
      st = fc;
    } else {
      st = first_max_combine(st, fc);
    }
  }
  idx[row] = (sj == (int)n - 1) ? (uint32_t)sj : st.i;
}
