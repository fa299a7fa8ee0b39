// bf16 GEMM, aligned shapes (M % 256 == 0, N % 256 == 0, K % 64 == 0):
// direct global->LDS loads and LDS transpose reads on gfx950.
//
// Semantics and order are those of gemm_bf16.hip (the reference's
// f32.matmul.row-major.materialize contraction, catena-lang/stdlib/
// matrix.hex:236-327, on bf16 inputs widened exactly, f32 accumulation, NN
// row-major).  Fixed order: one workgroup owns each 256x256 output tile, the
// K loop runs ascending in BK = 64 slabs of two k32 MFMA steps, no split-K and
// no atomics, so results are bitwise identical run to run.
//
// Data movement:
//  * Every 16-byte chunk of the A and B slabs goes global -> LDS with
//    global_load_lds_dwordx4 (no VGPR staging).  One instruction writes 1 KiB
//    of LDS contiguously (lane l -> base + 16 l), so bank-conflict freedom on
//    the read side comes from an XOR swizzle chosen through the global
//    address each lane fetches:
//      A slab [256 rows][128 B]: LDS chunk p of row r holds global chunk
//        p ^ hA(r), hA(r) = (r >> 1) & 7;
//      B slab [64 k][512 B]:     LDS chunk p of row k holds global chunk
//        p ^ hB(k), hB(k) = 2 * ((k & 3) | ((k >> 3) & 1) << 2).
//  * A fragments: one ds_read_b128 per 16x32 block (lane 16G+m reads 8
//    consecutive k of row m starting at 8G).
//  * B fragments: two ds_read_b64_tr_b16 per 32x16 block.  Within a 16-lane
//    group, lane i of the transpose read receives element i%4 of the 8-byte
//    chunks addressed by lanes 4j + i/4 (j = 0..3); lane s of group G
//    addresses row kk + 8G + 4h + s/4, columns nb + 4(s%4) .. +3, so lane i
//    receives 4 consecutive k of column nb + i, matching A's k order.
//  * The MFMA computes C^T blocks (B fragment as the first operand) so each
//    lane ends with 4 consecutive output columns of one row: 8-byte (bf16)
//    or 16-byte (f32) stores.
// Waves: 8 per workgroup (2 per SIMD), wave tile 128 x 64 (wm = wave / 4,
// wn = wave % 4), 8 x 4 accumulator blocks = 128 accumulator registers, so
// the second wave on each SIMD can issue while the first waits on LDS.
// Pipeline: two LDS stages (2 x 64 KiB); slab t+1's loads are in flight while
// slab t is multiplied; a stage is refilled only after a barrier that follows
// the last read of it.  One barrier per slab; the fragments of the next k32
// step are read from LDS during the current step's MFMAs, one read per MFMA
// over the first 16 of its 32 MFMAs.  This kernel serves aligned tiles with
// K % 128 != 0 (the four-stage k32 kernels need whole groups of four 32-k
// slabs).
#include "common.h"

namespace {
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int A_STAGE = BM * BK;  // elements
constexpr int B_STAGE = BK * BN;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

CATENA_DEV uint32_t hA(uint32_t r) { return (r >> 1) & 7u; }
CATENA_DEV uint32_t hB(uint32_t k) { return 2u * ((k & 3u) | (((k >> 3) & 1u) << 2)); }

CATENA_DEV bf16x8_t cat_bf16(i16x4_t lo, i16x4_t hi) {
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

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

// s_waitcnt with only vmcnt constrained (gfx9 encoding: vmcnt[3:0] and
// vmcnt[5:4] at bits 15:14, expcnt and lgkmcnt left at their maxima).
#define CATENA_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0070 | 0x0F00)

template <bool OUT_BF16>
CATENA_DEV void gemm_lds_body(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                              void* __restrict__ C, uint64_t M, uint64_t N, uint64_t K) {
  extern __shared__ __attribute__((aligned(1024))) uint16_t smem[];
  uint16_t* As = smem;                // [2][A_STAGE]
  uint16_t* Bs = smem + 2 * A_STAGE;  // [2][B_STAGE]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;  // 0..7
  const int wm = wave >> 2, wn = wave & 3;

  const uint32_t tiles_m = (uint32_t)(M / BM), tiles_n = (uint32_t)(N / BN);
  uint32_t tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;

  // Per-lane byte offsets of this wave's 4 A and 4 B load instructions (a
  // slab is 32 + 32 one-KiB instructions spread over the 8 waves), relative
  // to the slab's uniform base; 32 bits suffice (256 rows of A, 64 of B).
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t r = 32 * wave + 8 * i + (lane >> 3);
    const uint32_t q = (uint32_t)(lane & 7) ^ hA(r);
    aoff[i] = (uint32_t)((r * K + 8 * q) * 2);
    const uint32_t kr = 8 * wave + 2 * i + (lane >> 5);
    const uint32_t qb = (uint32_t)(lane & 31) ^ hB(kr);
    boff[i] = (uint32_t)((kr * N + 8 * qb) * 2);
  }
  const char* abase = reinterpret_cast<const char*>(A + m0 * K);
  const char* bbase = reinterpret_cast<const char*>(B + n0);
  auto issue = [&](uint64_t slab, int stage) {
    const uint64_t k0 = slab * BK;
    const char* ab = abase + k0 * 2;
    const char* bb = bbase + k0 * N * 2;
    uint16_t* as = As + stage * A_STAGE + (32 * wave) * BK;
    uint16_t* bs = Bs + stage * B_STAGE + (8 * wave) * BN;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(ab + aoff[i], (lds_void*)(as + 8 * i * BK), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(bb + boff[i], (lds_void*)(bs + 2 * i * BN), 16, 0, 0);
  };

  f32x4_t acc[8][4];  // [row block i][col block j], transposed blocks
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const uint64_t nk = K / BK;
  issue(0, 0);
  if (nk > 1) issue(1, 1);

  // Fragment addressing (byte offsets inside a stage).  For A, hA(row) is
  // the same for the 8 row blocks of a lane (16 rows apart), so one base
  // plus immediates covers them.  For B, hB(row) is the same for both k32
  // steps and both halves of a fragment, so 4 offsets (one per column block)
  // cover every read.
  const int G = lane >> 4, s = lane & 15;
  const uint32_t a_row0 = wm * 128 + s;
  const uint32_t a_lds = a_row0 * BK * 2 + 16 * ((uint32_t)G ^ hA(a_row0));  // + 16*16*BK*i, ^(kk/8) below
  const uint32_t b_krow = 8 * G + (s >> 2);
  const uint32_t hb = hB(b_krow);
  uint32_t b_lds[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t col = wn * 64 + 16 * j + 4 * (s & 3);
    b_lds[j] = b_krow * BN * 2 + 16 * ((col >> 3) ^ hb) + 2 * (col & 7);
  }

  struct Frags {
    bf16x8_t a[8];
    bf16x8_t b[4];
  };
  // LDS -> registers for one k32 step of this wave's 128 x 64 block.
  auto load_frags = [&](int stage, int kk, Frags& f) {
    const char* as = reinterpret_cast<const char*>(As + stage * A_STAGE);
    const char* bs = reinterpret_cast<const char*>(Bs + stage * B_STAGE);
    // A chunk index for this kk is (kk/8 + G) ^ hA = (G ^ hA) ^ (kk/8): kk/8
    // is 0 or 4 and hA < 8, so the XOR with kk/8 flips bit 2 of the chunk.
    const uint32_t a_off = kk == 0 ? a_lds : (a_lds ^ (4u * 16u));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      f.a[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(as + a_off + i * 16 * BK * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const char* p = bs + b_lds[j] + kk * BN * 2;
      i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
      i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * BN * 2));
      f.b[j] = cat_bf16(lo, hi);
    }
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };

  // LDS reads of `next` interleaved with the MFMAs of `cur`, pinned with
  // scheduling barriers so that few reads are outstanding when an MFMA
  // issues (the LDS counter tracks only 15 operations, so a block of 16
  // reads ahead of the MFMAs forces a full wait): one read per MFMA over the
  // first 16 MFMAs, then 16 MFMAs with no reads (the reads have landed by
  // the next barrier).
  auto load_mma = [&](int stage, int kk, Frags& next, const Frags& cur) {
    const char* as = reinterpret_cast<const char*>(As + stage * A_STAGE);
    const char* bs = reinterpret_cast<const char*>(Bs + stage * B_STAGE);
    const uint32_t a_off = kk == 0 ? a_lds : (a_lds ^ (4u * 16u));
    i16x4_t blo[4], bhi[4];
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      if (g < 8) {
        next.a[g] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(as + a_off + g * 16 * BK * 2));
      } else {
        const int j = (g - 8) >> 1;
        const char* p = bs + b_lds[j] + kk * BN * 2;
        if ((g & 1) == 0)
          blo[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
        else
          bhi[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * BN * 2));
      }
      const int j = g >> 3, i = g & 7;
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int m = 16; m < 32; ++m) {
      const int j = m >> 3, i = m & 7;
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);   // sixteen MFMAs
#pragma unroll
    for (int j = 0; j < 4; ++j) next.b[j] = cat_bf16(blo[j], bhi[j]);
  };

  // one barrier per slab; the fragments of the next k32 step are read from
  // LDS while the current step's MFMAs run:
  //   read F1 (2nd half of slab it) | MFMA F0 | wait: F1 landed, my slab it+1
  //   loads landed | barrier | refill this stage with slab it+2 | read F0 (1st
  //   half of slab it+1) | MFMA F1
  if (nk > 1) {
    CATENA_WAIT_VMCNT(8);
  } else {
    CATENA_WAIT_VMCNT(0);
  }
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  Frags f0, f1;
  load_frags(0, 0, f0);
  for (uint64_t it = 0; it + 1 < nk; ++it) {
    const int stage = (int)(it & 1);
    load_mma(stage, 32, f1, f0);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): f1 has landed
    CATENA_WAIT_VMCNT(0);                // this wave's slab it+1 has landed
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (it + 2 < nk) issue(it + 2, stage);
    load_mma(stage ^ 1, 0, f0, f1);
  }
  load_mma((int)((nk - 1) & 1), 32, f1, f0);
  mma(f1);

  // acc[i][j] lane (G, s) holds C[row = 16 i + s][cols 16 j + 4G .. +3] of
  // the wave's 128 x 64 block.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint64_t gr = m0 + wm * 128 + 16 * i + s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint64_t gc = n0 + wn * 64 + 16 * j + 4 * G;
      const f32x4_t v = acc[i][j];
      if (OUT_BF16) {
        uint2 p;
        p.x = pack_bf16x2(v[0], v[1]);
        p.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2*>(static_cast<uint16_t*>(C) + gr * N + gc) = p;
      } else {
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(C) + gr * N + gc) = v;
      }
    }
  }
}
}  // namespace

#define CATENA_GEMM_LDS_KERNEL(NAME, OUTB)                                                \
  extern "C" __global__ __launch_bounds__(512) void NAME(                                 \
      const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, \
      uint64_t M, uint64_t N, uint64_t K) {                                               \
    gemm_lds_body<OUTB>(A, B, C, M, N, K);                                                \
  }

CATENA_GEMM_LDS_KERNEL(catena_gemm_bf16_lds_bf16out, true)
CATENA_GEMM_LDS_KERNEL(catena_gemm_bf16_lds_f32out, false)
