// Decode-shape bf16 GEMM: Y[M x N] = X[M x K] * W[K x N] for M <= 16.
//
// Same contraction as gemm_bf16.hip (catena-lang/stdlib/matrix.hex:236-327,
// NN row-major, bf16 widened exactly, f32 accumulation) but shaped for the
// decode step, where W dominates the traffic (2*N*K bytes against 2*M*K for
// X) and the kernel is HBM-bound.  All 16 MFMA rows are X's (rows >= M are
// zero), so one v_mfma_f32_16x16x32_bf16 consumes a 32(k) x 16(n) piece of W.
//
// Work split (fixed, data independent):
//   * a wave owns 128 consecutive columns and a contiguous chunk of KW k;
//   * a workgroup holds 4 waves on 4 consecutive k chunks and adds their
//     partials in ascending chunk order through LDS;
//   * grid.y = number of such k groups (S).  S == 1 writes Y (bf16 or f32)
//     directly; otherwise each workgroup writes an f32 partial P[s][m][n]
//     and catena_gemm_bf16_decode_reduce adds them in ascending s.
// No atomics; the addition order depends only on the shape, so results are
// bitwise identical run to run.
//
// Lane mapping: lane l = 16*g + c.  For a k32 step at k0 the lane loads the
// 8x8 bf16 block W[k0+8g .. k0+8g+7][n0+8c .. n0+8c+7] (8 x 16 B; per load
// instruction the 16 lanes of a g read 256 contiguous bytes), transposes it
// in registers, and feeds column n0+8c+j as the B operand of MFMA number j.
// MFMA j's output column c therefore maps to global column n0 + 8c + j, so
// each lane ends up holding 8 consecutive columns of 4 rows: stores are
// 16-byte (bf16) / 32-byte (f32) runs.
#include "common.h"

namespace {
constexpr int COLS_PER_WAVE = 128;

CATENA_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

CATENA_DEV void transpose8x8(const u32x4_t in[8], u32x4_t out[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      uint32_t x = in[2 * p][j / 2], y = in[2 * p + 1][j / 2];
      w[p] = (j & 1) ? ((x >> 16) | (y & 0xFFFF0000u)) : ((x & 0xFFFFu) | (y << 16));
    }
    out[j] = u32x4_t{w[0], w[1], w[2], w[3]};
  }
}

CATENA_DEV void load_w(const uint16_t* __restrict__ W, uint64_t K, uint64_t N, uint64_t k0,
                       uint64_t col, int g, u32x4_t r[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint64_t kr = k0 + 8 * g + i;
    if (kr < K && col < N)
      r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(W + kr * N + col));
    else
      r[i] = u32x4_t{0u, 0u, 0u, 0u};
  }
}
}  // namespace

// grid = (ceil(N/128), S), block = 256.  KW = k per wave (multiple of 32).
extern "C" __global__ __launch_bounds__(256) void catena_gemm_bf16_decode(
    const uint16_t* __restrict__ X, const uint16_t* __restrict__ W, void* __restrict__ Y,
    float* __restrict__ P, uint32_t M, uint64_t N, uint64_t K, uint32_t KW, uint32_t out_f32) {
  __shared__ f32x4_t red[3][8][64];  // partials of waves 1..3

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, c = lane & 15;
  const uint64_t n0 = (uint64_t)blockIdx.x * COLS_PER_WAVE;
  const uint64_t col = n0 + 8 * c;
  const uint64_t kbeg = ((uint64_t)blockIdx.y * 4 + wave) * KW;
  uint64_t kend = kbeg + KW;
  if (kend > K) kend = K;

  f32x4_t acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int xrow = lane & 15;
  const bool xlive = xrow < (int)M;
  if (kbeg < kend) {
    u32x4_t cur[8], nxt[8];
    load_w(W, K, N, kbeg, col, g, cur);
    for (uint64_t k0 = kbeg; k0 < kend; k0 += 32) {
      const bool more = k0 + 32 < kend;
      if (more) load_w(W, K, N, k0 + 32, col, g, nxt);
      const uint64_t xk = k0 + 8 * g;
      u32x4_t xa = u32x4_t{0u, 0u, 0u, 0u};
      if (xlive && xk < K) xa = *reinterpret_cast<const u32x4_t*>(X + (uint64_t)xrow * K + xk);
      u32x4_t bt[8];
      transpose8x8(cur, bt);
      const bf16x8_t af = as_bf16x8(xa);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, as_bf16x8(bt[j]), acc[j], 0, 0, 0);
      if (more) {
#pragma unroll
        for (int i = 0; i < 8; ++i) cur[i] = nxt[i];
      }
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) red[wave - 1][j][lane] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f32x4_t o = red[w][j][lane];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[j][q] = acc[j][q] + o[q];
    }

  // lane holds rows 4g+q, columns n0 + 8c + j (j = 0..7)
  if (col >= N) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint32_t row = 4 * g + q;
    if (row >= M) continue;
    if (gridDim.y == 1 && !out_f32) {
      u32x4_t packed = u32x4_t{pack_bf16x2(acc[0][q], acc[1][q]), pack_bf16x2(acc[2][q], acc[3][q]),
                               pack_bf16x2(acc[4][q], acc[5][q]), pack_bf16x2(acc[6][q], acc[7][q])};
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(Y) + (uint64_t)row * N + col) = packed;
    } else {
      // S == 1 with f32 output writes Y itself; otherwise partial s of P
      float* dst = gridDim.y == 1 ? static_cast<float*>(Y) + (uint64_t)row * N + col
                                  : P + ((uint64_t)blockIdx.y * M + row) * N + col;
      *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{acc[0][q], acc[1][q], acc[2][q], acc[3][q]};
      *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{acc[4][q], acc[5][q], acc[6][q], acc[7][q]};
    }
  }
}

// Y[m][n] = P[0][m][n] + P[1][m][n] + ... + P[S-1][m][n], ascending s, then
// bf16 (RNE) unless out_f32.
extern "C" __global__ __launch_bounds__(256) void catena_gemm_bf16_decode_reduce(
    const float* __restrict__ P, void* __restrict__ Y, uint32_t M, uint64_t N, uint32_t S,
    uint32_t out_f32) {
  const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // over M*N/4
  const uint64_t total = (uint64_t)M * N / 4;
  if (idx >= total) return;
  const f32x4_t* p4 = reinterpret_cast<const f32x4_t*>(P);
  f32x4_t acc = p4[idx];
  for (uint32_t s = 1; s < S; ++s) {
    f32x4_t v = p4[(uint64_t)s * total + idx];
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = acc[q] + v[q];
  }
  if (out_f32) {
    reinterpret_cast<f32x4_t*>(Y)[idx] = acc;
    return;
  }
  uint2 out;
  out.x = pack_bf16x2(acc[0], acc[1]);
  out.y = pack_bf16x2(acc[2], acc[3]);
  reinterpret_cast<uint2*>(Y)[idx] = out;
}
