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

// 16 k values of the cell's row of A and column of B (k-contiguous in LDS)
CATENA_DEV void read16(float4 (&a)[4], float4 (&b)[4], const float* ar, const float* br) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    a[u] = *reinterpret_cast<const float4*>(ar + 4 * u);
    b[u] = *reinterpret_cast<const float4*>(br + 4 * u);
  }
}

// acc = acc + fl(a_k * b_k) for the 16 k values in ascending order
CATENA_DEV float fold16(float acc, const float4 (&a)[4], const float4 (&b)[4]) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    float prod = a[u].x * b[u].x;
    acc = acc + prod;
    prod = a[u].y * b[u].y;
    acc = acc + prod;
    prod = a[u].z * b[u].z;
    acc = acc + prod;
    prod = a[u].w * b[u].w;
    acc = acc + prod;
  }
  return acc;
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
    // only the kt live k values enter the chain, in ascending order; the
    // LDS reads of the next 16 k are issued before the current 16 are
    // folded, so their latency sits under the chain instead of in front of it
    int kk = 0;
    // (two register sets in turn: set 0 holds k kk .. kk + 15 at the top of
    // each pass)
    if (kt >= 16) {
      float4 a0[4], b0[4], a1[4], b1[4];
      read16(a0, b0, &As[ty][0], &Bs[tx][0]);
      // (the scheduling barriers keep each set's reads in front of the other
      // set's fold; left alone the compiler moves them down to their use)
      for (; kk + 48 <= kt; kk += 32) {
        read16(a1, b1, &As[ty][kk + 16], &Bs[tx][kk + 16]);
        __builtin_amdgcn_sched_barrier(0);
        acc = fold16(acc, a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        read16(a0, b0, &As[ty][kk + 32], &Bs[tx][kk + 32]);
        __builtin_amdgcn_sched_barrier(0);
        acc = fold16(acc, a1, b1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (kk + 32 <= kt) {
        read16(a1, b1, &As[ty][kk + 16], &Bs[tx][kk + 16]);
        __builtin_amdgcn_sched_barrier(0);
        acc = fold16(acc, a0, b0);
        acc = fold16(acc, a1, b1);
        kk += 32;
      } else {
        acc = fold16(acc, a0, b0);
        kk += 16;
      }
    }
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

// The same contraction for small outputs with k % 16 == 0 and 16-byte
// aligned rows of B (m % 4 == 0), again on 16 x 16 tiles with one cell per
// thread (256^3: 256 workgroups), but with A kept out of LDS: wave w owns
// rows 16 blockIdx.y + 4 w + r, r = lane / 16, and lane l column
// 16 blockIdx.x + l % 16, so a row of A is uniform within each 16-lane DPP
// row.  For a 16-k group lane 16 r + q holds A[row r][k0 + q] (one 4-byte
// buffer load) and the multiply takes it through a DPP row broadcast
// (v_mul_f32_dpp row_newbcast:q), no instruction of its own: a broadcast
// LDS read costs the shared LDS more than the multiply-add it feeds.  The B
// tile of a chunk of 256 k (16 columns, 16 KB) goes through LDS, requested
// at once with one 16-byte buffer load per thread and 64 k, and is folded
// after one barrier, each 16-k group's B reads issued before the previous
// group is folded; each group's 16 products are formed before its 16
// dependent adds (one wave per SIMD: nothing else fills the wait when an
// add follows its own multiply).  Each cell's chain is the one above:
// acc = +0, then for kk ascending acc = acc + fl(A[i,kk] * B[kk,j]).
namespace {
constexpr int Q_T = 16, Q_KC = 256;

// acc = acc + fl(A_k * b_k) for 16 k in ascending order, A_k in lane k % 16
// of every row of ra: the 16 products first, then the 16 dependent adds
// (with one wave per SIMD nothing else fills the wait when each add follows
// its own multiply)
CATENA_DEV float fold16_row_bcast(float acc, float ra, const float (&b)[16]) {
  float prod[16];
  prod[0] = row_bcast16<0>(ra) * b[0];
  prod[1] = row_bcast16<1>(ra) * b[1];
  prod[2] = row_bcast16<2>(ra) * b[2];
  prod[3] = row_bcast16<3>(ra) * b[3];
  prod[4] = row_bcast16<4>(ra) * b[4];
  prod[5] = row_bcast16<5>(ra) * b[5];
  prod[6] = row_bcast16<6>(ra) * b[6];
  prod[7] = row_bcast16<7>(ra) * b[7];
  prod[8] = row_bcast16<8>(ra) * b[8];
  prod[9] = row_bcast16<9>(ra) * b[9];
  prod[10] = row_bcast16<10>(ra) * b[10];
  prod[11] = row_bcast16<11>(ra) * b[11];
  prod[12] = row_bcast16<12>(ra) * b[12];
  prod[13] = row_bcast16<13>(ra) * b[13];
  prod[14] = row_bcast16<14>(ra) * b[14];
  prod[15] = row_bcast16<15>(ra) * b[15];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = 0; q < 16; ++q) acc = acc + prod[q];
  return acc;
}

// k 16 g .. 16 g + 15 of this lane's B column (row stride 16 floats)
CATENA_DEV void q16_read16(float (&b)[16], const float* bs) {
#pragma unroll
  for (int q = 0; q < 16; ++q) b[q] = bs[q * Q_T];
}
}  // namespace

// LDS: Q_KC * Q_T * 4 bytes (dynamic).
extern "C" __global__ __launch_bounds__(256) void catena_gemm_f32_exact_q16(
    const float* __restrict__ A, const float* __restrict__ B, float* __restrict__ C,
    uint64_t n, uint64_t m, uint64_t k) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const uint64_t row0 = (uint64_t)blockIdx.y * Q_T, col0 = (uint64_t)blockIdx.x * Q_T;
  const uint64_t arow = row0 + 4 * wave + (lane >> 4);
  const uint64_t ccol = col0 + (lane & 15);
  // buffer loads with 32-bit byte offsets (the host keeps (n + 16) k 4 and
  // (k + 256) m 4 below 2^31): a read past either matrix returns 0; a B
  // read past column m reads the next row.  Neither value is folded into a
  // stored cell.
  const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, (int)(n * k * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc((void*)B, (short)0, (int)(k * m * 4), 0x00020000);
  const uint32_t m4 = (uint32_t)m * 4u;
  const float* bs = reinterpret_cast<const float*>(smem) + (lane & 15);
  float acc = __uint_as_float(0u);
  for (uint64_t c0 = 0; c0 < k; c0 += Q_KC) {
    const int ng = (k - c0) < (uint64_t)Q_KC ? (int)((k - c0) / 16) : Q_KC / 16;
    // B copy u of thread t: chunk row 64 u + t / 4, columns 4 (t % 4) .. + 3;
    // A group g: row arow, k 16 g + l % 16 of the chunk
    const uint32_t bvo = (uint32_t)(((c0 + tid / 4) * m + col0 + 4 * (tid % 4)) * 4);
    const uint32_t avo = (uint32_t)((arow * k + c0 + (lane & 15)) * 4);
    float4 rb[4];
    float ra[Q_KC / 16];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (64 * u < 16 * ng)
        rb[u] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(brs, (int)bvo, (int)((uint32_t)(64 * u) * m4), 0));
#pragma unroll
    for (int g = 0; g < Q_KC / 16; ++g)
      if (g < ng) ra[g] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ars, (int)(avo + 64u * g), 0, 0));
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (64 * u < 16 * ng) *reinterpret_cast<float4*>(smem + (256 * u + tid) * 16) = rb[u];
    __syncthreads();
    // 16-k groups, two register sets in turn, each group's B reads issued
    // before the previous group is folded
    float b0[16], b1[16];
    q16_read16(b0, bs);
#pragma unroll
    for (int g = 0; g < Q_KC / 16; g += 2) {
      if (g < ng) {
        if (g + 1 < ng) q16_read16(b1, bs + (16 * (g + 1)) * Q_T);
        __builtin_amdgcn_sched_barrier(0);
        acc = fold16_row_bcast(acc, ra[g], b0);
        __builtin_amdgcn_sched_barrier(0);
        if (g + 1 < ng) {
          if (g + 2 < ng) q16_read16(b0, bs + (16 * (g + 2)) * Q_T);
          __builtin_amdgcn_sched_barrier(0);
          acc = fold16_row_bcast(acc, ra[g + 1], b1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    __syncthreads();
  }
  if (arow < n && ccol < m) C[arow * m + ccol] = acc;
}
