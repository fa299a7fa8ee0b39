// Exact-order f32 GEMM: the lowering of f32.matmul.row-major.materialize.
//
// Reference semantics (catena-lang/stdlib/matrix.hex:236-327 lowered by
// catena-lang/src/codegen/ops/materializec.rs:36-82 and
// catena-lang/src/codegen/ops/reducec.rs:73-130): for every output cell
// (i, j) of C[n x m] = A[n x k] * B[k x m] (both row-major, NN),
//     acc = +0.0f; for kk = 0 .. k-1 ascending: acc = acc + A[i,kk] * B[kk,j]
// with the multiply and the add separately rounded.  The reference runs one
// thread per cell that streams a row of A and a column of B from global
// memory.  Here a 64x64 output tile is staged through LDS 16 k-values at a
// time and every thread owns a 4x4 block of cells; each cell keeps its own
// k-ascending chain of v_mul_f32 then v_add_f32, so the result is bitwise the
// reference's.  No split-K, no atomics.
#include "common.h"

namespace {
constexpr int TM = 64, TN = 64, TK = 16;
}

extern "C" __global__ __launch_bounds__(256) void catena_gemm_f32_exact(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    uint64_t n, uint64_t m, uint64_t k) {
  __shared__ float As[TK][TM + 1];
  __shared__ float Bs[TK][TN];

  const int tid = threadIdx.x;
  const int tx = tid % 16;  // column group: cols tx + 16*jj
  const int ty = tid / 16;  // row group: rows ty + 16*ii
  const uint64_t row0 = (uint64_t)blockIdx.y * TM;
  const uint64_t col0 = (uint64_t)blockIdx.x * TN;

  float acc[4][4];
#pragma unroll
  for (int ii = 0; ii < 4; ++ii)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[ii][jj] = __uint_as_float(0u);

  for (uint64_t k0 = 0; k0 < k; k0 += TK) {
    const int kt = (k - k0) < (uint64_t)TK ? (int)(k - k0) : TK;
    // A tile: 64 rows x 16 k (row-major in A) -> As[kk][row]
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int idx = tid + 256 * e;  // 0..1023
      int r = idx / TK, kk = idx % TK;
      uint64_t gi = row0 + r;
      float v = 0.0f;
      if (gi < n && kk < kt) v = A[gi * k + k0 + kk];
      As[kk][r] = v;
    }
    // B tile: 16 k x 64 cols -> Bs[kk][col]
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int idx = tid + 256 * e;
      int kk = idx / TN, c = idx % TN;
      uint64_t gj = col0 + c;
      float v = 0.0f;
      if (gj < m && kk < kt) v = B[(k0 + kk) * m + gj];
      Bs[kk][c] = v;
    }
    __syncthreads();
    // Only the kt live k-values are folded: the chain sees exactly
    // k = 0 .. k-1 in ascending order.
    for (int kk = 0; kk < kt; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) a[ii] = As[kk][ty + 16 * ii];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) b[jj] = Bs[kk][tx + 16 * jj];
#pragma unroll
      for (int ii = 0; ii < 4; ++ii)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          float prod = a[ii] * b[jj];
          acc[ii][jj] = acc[ii][jj] + prod;
        }
    }
    __syncthreads();
  }

#pragma unroll
  for (int ii = 0; ii < 4; ++ii) {
    uint64_t gi = row0 + ty + 16 * ii;
    if (gi >= n) continue;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      uint64_t gj = col0 + tx + 16 * jj;
      if (gj < m) C[gi * m + gj] = acc[ii][jj];
    }
  }
}
