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

// The same contraction for small outputs, where 64x64 tiles would leave most
// CUs idle (256^3 is 16 tiles of 64x64 on a 256-CU device): a 16x16 output
// tile per workgroup of 256 threads, one cell per thread, so 256^3 launches
// 256 workgroups.  A 16-row x 128-k slab of A and a 128-k x 16-column slab of
// B are staged in LDS k-contiguous per row / per column ([row][k] and
// [col][k], rows padded by 4 floats), so each thread reads the next four k
// values of its row and of its column with one 16-byte read each.  Every
// global load is issued unconditionally from an in-range address (element 0
// stands in for one past the edge, and its value is replaced by 0), so the
// slab's 16 loads per thread are in flight together, and the next slab is
// requested into registers before the current one is folded.  The cell's
// chain is the one above: acc = +0, then for kk ascending
// acc = acc + fl(A[i,kk] * B[kk,j]), separately rounded -- bitwise the same
// result as the 64x64 instance and the reference.
namespace {
constexpr int S_T = 16, S_K = 128, S_PAD = 4;

struct Slab {
  float a[8], b[8];
  uint32_t live;  // bit e: a[e] in range, bit 8 + e: b[e] in range
};

// thread tid's share of the slab at k0: A row tid / 16, k 8 (tid % 16) .. +7;
// B k (tid + 256 e) / 16, column (tid + 256 e) % 16 for e = 0 .. 7.  The
// out-of-range values are zeroed when the slab is stored, not here, so no
// instruction waits on the loads until then.
CATENA_DEV void load_slab(Slab& sl, const float* __restrict__ A, const float* __restrict__ B,
                          uint64_t n, uint64_t m, uint64_t k, uint64_t row0, uint64_t col0,
                          uint64_t k0, int tid) {
  const int r = tid / 16, q = tid % 16;
  const uint64_t gi = row0 + r;
  uint32_t live = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint64_t kk = k0 + 8 * q + e;
    const bool ok = gi < n && kk < k;
    sl.a[e] = A[ok ? gi * k + kk : 0];
    live |= (ok ? 1u : 0u) << e;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int idx = tid + 256 * e;
    const uint64_t kk = k0 + idx / S_T, gj = col0 + idx % S_T;
    const bool ok = gj < m && kk < k;
    sl.b[e] = B[ok ? kk * m + gj : 0];
    live |= (ok ? 1u : 0u) << (8 + e);
  }
  sl.live = live;
}

CATENA_DEV float live_or_zero(float v, uint32_t live, int bit) {
  return (live >> bit) & 1u ? v : 0.0f;
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void catena_gemm_f32_exact_t16(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    uint64_t n, uint64_t m, uint64_t k) {
  __shared__ __align__(16) float As[S_T][S_K + S_PAD];
  __shared__ __align__(16) float Bs[S_T][S_K + S_PAD];

  const int tid = threadIdx.x;
  const int tx = tid % S_T;  // column of the cell
  const int ty = tid / S_T;  // row of the cell
  const uint64_t row0 = (uint64_t)blockIdx.y * S_T;
  const uint64_t col0 = (uint64_t)blockIdx.x * S_T;

  float acc = __uint_as_float(0u);
  Slab sl;
  if (k > 0) load_slab(sl, A, B, n, m, k, row0, col0, 0, tid);
  for (uint64_t k0 = 0; k0 < k; k0 += S_K) {
    const int kt = (k - k0) < (uint64_t)S_K ? (int)(k - k0) : S_K;
    {
      const int r = tid / 16, q = tid % 16;
      float a[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) a[e] = live_or_zero(sl.a[e], sl.live, e);
      *reinterpret_cast<float4*>(&As[r][8 * q]) = make_float4(a[0], a[1], a[2], a[3]);
      *reinterpret_cast<float4*>(&As[r][8 * q + 4]) = make_float4(a[4], a[5], a[6], a[7]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = tid + 256 * e;
        Bs[idx % S_T][idx / S_T] = live_or_zero(sl.b[e], sl.live, 8 + e);
      }
    }
    __syncthreads();
    if (k0 + S_K < k) load_slab(sl, A, B, n, m, k, row0, col0, k0 + S_K, tid);
    // only the kt live k values enter the chain, in ascending order
    int kk = 0;
#pragma unroll 4
    for (; kk + 4 <= kt; kk += 4) {
      const float4 a = *reinterpret_cast<const float4*>(&As[ty][kk]);
      const float4 b = *reinterpret_cast<const float4*>(&Bs[tx][kk]);
      float prod = a.x * b.x;
      acc = acc + prod;
      prod = a.y * b.y;
      acc = acc + prod;
      prod = a.z * b.z;
      acc = acc + prod;
      prod = a.w * b.w;
      acc = acc + prod;
    }
    for (; kk < kt; ++kk) {
      const float prod = As[ty][kk] * Bs[tx][kk];
      acc = acc + prod;
    }
    __syncthreads();
  }
  const uint64_t gi = row0 + ty, gj = col0 + tx;
  if (gi < n && gj < m) C[gi * m + gj] = acc;
}
