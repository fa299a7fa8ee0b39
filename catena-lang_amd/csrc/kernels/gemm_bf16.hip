// bf16 GEMM on gfx950 MFMA with a fixed, data-independent reduction order:
// the general-shape (edge) kernel, for shapes the aligned tile kernels do not
// take (M or N not a multiple of 256, K not a multiple of 64, unaligned
// pointers).  Every load and store is bounds-checked; out-of-range A and B
// elements read as +0.
//
// Semantics: the reference's f32.matmul.row-major.materialize contraction
// (catena-lang/stdlib/matrix.hex:236-327; NN, both operands row-major:
// A[i,kk] = a[i*K+kk], B[kk,j] = b[kk*N+j], catena-lang/src/codegen/ops/
// row_major.rs:9-28) applied to bf16 inputs widened exactly to f32, with f32
// accumulation and one RNE rounding to bf16 at the end (or f32 output).
// bf16 x bf16 products are exact in f32; the summation order is the MFMA
// datapath's, which differs from the reference's sequential fold, so parity
// against the sequential oracle is a stated error bound.  The order is fixed:
// every output tile is owned by one workgroup, the K loop runs ascending in
// BK=64 slabs, each slab is two v_mfma_f32_16x16x32_bf16 steps in ascending
// k, there is no split-K and no atomic, so results are bitwise identical run
// to run.
//
// Tiling: 256x256 output tile per workgroup of 256 threads (4 waves, 2x2),
// each wave owns 128x128 = 8x8 MFMA 16x16 blocks.  A and B slabs are
// double-buffered in LDS (2 x 2 x 256 x 72 bf16 = 144 KiB of gfx950's
// 160 KiB); the next slab's global loads are issued before the current
// slab's MFMAs.  B arrives N-contiguous, but the MFMA B operand wants 8
// consecutive k per lane, so each thread transposes an 8x8 bf16 block in
// registers before writing it to LDS k-contiguous.
#include "common.h"

namespace {
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int LDK = BK + 8;  // padded row (in bf16): 144 B, conflict-free b128 reads
constexpr int TILE_ELEMS = BM * LDK;

CATENA_DEV bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// Workgroup -> output tile.  Dispatch places consecutive workgroup ids on
// consecutive XCDs (8 on MI355X), each with its own L2.  The ids are first
// regrouped so that each XCD receives a contiguous range, then that range is
// walked in groups of GROUP_M tile rows, so the workgroups sharing an XCD
// share A row panels and B column panels.
CATENA_DEV void tile_of(uint32_t bid, uint32_t tiles_m, uint32_t tiles_n, uint32_t& tm,
                        uint32_t& tn) {
  const uint32_t total = tiles_m * tiles_n;
  if (total % 8u == 0u) bid = (bid % 8u) * (total / 8u) + bid / 8u;
  const uint32_t GROUP_M = 4;
  const uint32_t in_group = GROUP_M * tiles_n;
  const uint32_t group = bid / in_group;
  const uint32_t first_m = group * GROUP_M;
  const uint32_t gsize = (tiles_m - first_m) < GROUP_M ? (tiles_m - first_m) : GROUP_M;
  const uint32_t r = bid % in_group;
  tm = first_m + r % gsize;
  tn = r / gsize;
}

CATENA_DEV u32x4_t load_a_chunk(const uint16_t* __restrict__ A, uint64_t M, uint64_t K,
                                uint64_t row, uint64_t col) {
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint32_t lo = 0, hi = 0;
    if (row < M && col + 2 * h < K) lo = A[row * K + col + 2 * h];
    if (row < M && col + 2 * h + 1 < K) hi = A[row * K + col + 2 * h + 1];
    w[h] = lo | (hi << 16);
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

CATENA_DEV u32x4_t load_b_chunk(const uint16_t* __restrict__ B, uint64_t K, uint64_t N,
                                uint64_t row, uint64_t col) {
  uint32_t w[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint32_t lo = 0, hi = 0;
    if (row < K && col + 2 * h < N) lo = B[row * N + col + 2 * h];
    if (row < K && col + 2 * h + 1 < N) hi = B[row * N + col + 2 * h + 1];
    w[h] = lo | (hi << 16);
  }
  return u32x4_t{w[0], w[1], w[2], w[3]};
}

// 8x8 transpose of bf16: in[r] holds row r (8 n-values), out[j] holds
// column j (8 k-values, k-pairs packed low/high).
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

template <bool OUT_BF16>
CATENA_DEV void gemm_bf16_body(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                               void* __restrict__ C, uint64_t M, uint64_t N, uint64_t K) {
  extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
  uint16_t* As = smem;                  // [2][BM][LDK]
  uint16_t* Bs = smem + 2 * TILE_ELEMS;  // [2][BN][LDK], k-contiguous per column

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const uint32_t tiles_m = (uint32_t)((M + BM - 1) / BM);
  const uint32_t tiles_n = (uint32_t)((N + BN - 1) / BN);
  uint32_t tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;

  // A loader: chunk idx = tid + 256*e -> row idx/8, 8-col chunk idx%8
  // B loader: thread owns the 8x8 block (k-block kb, n-block nb)
  const int kb = tid & 7, nb = tid >> 3;

  u32x4_t ra[8], rb[8];
  auto gload = [&](uint64_t k0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int idx = tid + 256 * e;
      ra[e] = load_a_chunk(A, M, K, m0 + (idx >> 3), k0 + (idx & 7) * 8);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) rb[r] = load_b_chunk(B, K, N, k0 + kb * 8 + r, n0 + nb * 8);
  };
  auto lstore = [&](int buf) {
    uint16_t* as = As + buf * TILE_ELEMS;
    uint16_t* bs = Bs + buf * TILE_ELEMS;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int idx = tid + 256 * e;
      *reinterpret_cast<u32x4_t*>(as + (idx >> 3) * LDK + (idx & 7) * 8) = ra[e];
    }
    u32x4_t t[8];
    transpose8x8(rb, t);
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<u32x4_t*>(bs + (nb * 8 + j) * LDK + kb * 8) = t[j];
  };

  f32x4_t acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint64_t nk = (K + BK - 1) / BK;
  gload(0);
  lstore(0);
  __syncthreads();

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;
  for (uint64_t it = 0; it < nk; ++it) {
    const int cur = (int)(it & 1);
    if (it + 1 < nk) gload((it + 1) * BK);
    const uint16_t* as = As + cur * TILE_ELEMS + (wm * 128 + frag_row) * LDK + frag_k;
    const uint16_t* bs = Bs + cur * TILE_ELEMS + (wn * 128 + frag_row) * LDK + frag_k;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8_t af[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        af[i] = as_bf16x8(*reinterpret_cast<const u32x4_t*>(as + i * 16 * LDK + s * 32));
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        bf16x8_t bfr = as_bf16x8(*reinterpret_cast<const u32x4_t*>(bs + j * 16 * LDK + s * 32));
#pragma unroll
        for (int i = 0; i < 8; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr, acc[i][j], 0, 0, 0);
      }
    }
    if (it + 1 < nk) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 4*(lane/16)+q, column lane%16 of each block.
  const int ccol = lane & 15;
  const int crow = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint64_t gc = n0 + wn * 128 + j * 16 + ccol;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint64_t gr = m0 + wm * 128 + i * 16 + crow + q;
        if (gr >= M || gc >= N) continue;
        if (OUT_BF16)
          static_cast<uint16_t*>(C)[gr * N + gc] = (uint16_t)f32_to_bf16_bits(acc[i][j][q]);
        else
          static_cast<float*>(C)[gr * N + gc] = acc[i][j][q];
      }
    }
  }
}
}  // namespace

#define CATENA_GEMM_BF16_KERNEL(NAME, OUTB)                                            \
  extern "C" __global__ __launch_bounds__(256) void NAME(                            \
      const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, \
      uint64_t M, uint64_t N, uint64_t K) {                                          \
    gemm_bf16_body<OUTB>(A, B, C, M, N, K);                                          \
  }

CATENA_GEMM_BF16_KERNEL(catena_gemm_bf16_edge_bf16out, true)
CATENA_GEMM_BF16_KERNEL(catena_gemm_bf16_edge_f32out, false)
