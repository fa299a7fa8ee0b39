// bf16 GEMM, aligned shapes (M % 256 == 0, N % 256 == 0, K % 64 == 0, K >= 128): a
// deeper global->LDS pipeline than gemm_bf16_lds.hip for full-chip loads.
//
// Same contraction, tile and order as gemm_bf16_lds.hip (reference
// semantics: catena-lang/stdlib/matrix.hex:236-327 on bf16 inputs widened
// exactly, f32 accumulation, NN row-major): one workgroup per 256x256 output
// tile, 8 waves of 128x64, v_mfma_f32_16x16x32_bf16 with the B fragment as
// the first operand, K ascending in k32 steps, no split-K, no atomics.
//
// Pipeline: the K slab of one step is 32 wide (A [256][32] + B [32][256] =
// 32 KiB) and NS such stages live in LDS.  Fragments of step t+1 are read
// into registers while step t's MFMAs run, so at the barrier that opens step
// t+1 the stage of step t has already been consumed and is refilled at once
// with step t+NS.  Steps t+2 .. t+NS are then in flight (NS - 1 = 3 slabs,
// 96 KiB, with NS = 4 stages in 128 KiB of LDS), against one 64 KiB slab in
// the two-stage kernel.
// Swizzles (bank-conflict-free reads through the direct-to-LDS layout):
//   A stage [256][64 B]: LDS chunk p of row r holds global chunk p ^ ((r >> 2) & 3);
//   B stage [32][512 B]: LDS chunk p of row k holds global chunk p ^ hB(k),
//                        hB(k) = 2 * ((k & 3) | ((k >> 3) & 1) << 2).
#include "common.h"

namespace {
constexpr int BM = 256, BN = 256, BK = 32;
constexpr int A_STAGE = BM * BK;  // elements
constexpr int B_STAGE = BK * BN;
constexpr int STAGE = A_STAGE + B_STAGE;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

CATENA_DEV uint32_t hA(uint32_t r) { return (r >> 2) & 3u; }
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

#define CATENA_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt((((n) & 15) | (((n) >> 4) << 14)) | 0x0070 | 0x0F00)

template <bool OUT_BF16, int NS, bool FRONT>
CATENA_DEV void gemm_deep_body(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                               void* __restrict__ C, uint64_t M, uint64_t N, uint64_t K) {
  extern __shared__ __attribute__((aligned(1024))) uint16_t smem[];  // [NS][A_STAGE + B_STAGE]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;  // 0..7
  const int wm = wave >> 2, wn = wave & 3;

  const uint32_t tiles_m = (uint32_t)(M / BM), tiles_n = (uint32_t)(N / BN);
  uint32_t tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;

  // Loads per stage: A 16 KiB = 16 one-KiB instructions (16 rows of 64 B),
  // B 16 KiB = 16 instructions (2 rows of 512 B); 2 + 2 per wave.
  uint32_t aoff[2], boff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const uint32_t r = 32 * wave + 16 * i + (lane >> 2);
    const uint32_t q = (uint32_t)(lane & 3) ^ hA(r);
    aoff[i] = (uint32_t)((r * K + 8 * q) * 2);
    const uint32_t kr = 4 * wave + 2 * i + (lane >> 5);
    const uint32_t qb = (uint32_t)(lane & 31) ^ hB(kr);
    boff[i] = (uint32_t)((kr * N + 8 * qb) * 2);
  }
  const char* abase = reinterpret_cast<const char*>(A + m0 * K);
  const char* bbase = reinterpret_cast<const char*>(B + n0);
  auto issue = [&](uint64_t step, int stage) {
    const uint64_t k0 = step * BK;
    const char* ab = abase + k0 * 2;
    const char* bb = bbase + k0 * N * 2;
    uint16_t* as = smem + stage * STAGE + (32 * wave) * BK;
    uint16_t* bs = smem + stage * STAGE + A_STAGE + (4 * wave) * BN;
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(ab + aoff[i], (lds_void*)(as + 16 * i * BK), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_global_load_lds(bb + boff[i], (lds_void*)(bs + 2 * i * BN), 16, 0, 0);
  };

  f32x4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int G = lane >> 4, s = lane & 15;
  // A: row wm*128 + 16 i + s, chunk G ^ hA(row); hA is the same for all i
  const uint32_t a_lds = (wm * 128 + s) * BK * 2 + 16 * ((uint32_t)G ^ ((uint32_t)(s >> 2) & 3u));
  const uint32_t b_krow = 8 * G + (s >> 2);
  const uint32_t hb = hB(b_krow);
  uint32_t b_lds[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t col = wn * 64 + 16 * j + 4 * (s & 3);
    b_lds[j] = A_STAGE * 2 + b_krow * BN * 2 + 16 * ((col >> 3) ^ hb) + 2 * (col & 7);
  }

  struct Frags {
    bf16x8_t a[8];
    bf16x8_t b[4];
  };
  auto load_frags = [&](int stage, Frags& f) {
    const char* st = reinterpret_cast<const char*>(smem + stage * STAGE);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      f.a[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(st + a_lds + i * 16 * BK * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const char* p = st + b_lds[j];
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
  // Reads of `next` interleaved with the MFMAs of `cur`, pinned by
  // scheduling barriers.  FRONT: one read per MFMA over the first 16 MFMAs,
  // then 16 MFMAs with no reads, so the reads have landed by the barrier that
  // follows; otherwise one read per two MFMAs across the step.
  auto load_mma = [&](int stage, Frags& next, const Frags& cur) {
    const char* st = reinterpret_cast<const char*>(smem + stage * STAGE);
    i16x4_t blo[4], bhi[4];
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      if (g < 8) {
        next.a[g] = __builtin_bit_cast(
            bf16x8_t, *reinterpret_cast<const u32x4_t*>(st + a_lds + g * 16 * BK * 2));
      } else {
        const int j = (g - 8) >> 1;
        const char* p = st + b_lds[j];
        if ((g & 1) == 0)
          blo[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
        else
          bhi[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * BN * 2));
      }
      if (FRONT) {
        const int j = g >> 3, i = g & 7;
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int m = 2 * g + t, j = m >> 3, i = m & 7;
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
        }
      }
    }
    if (FRONT) {
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
    } else {
#pragma unroll
      for (int g = 0; g < 16; ++g) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // two MFMAs
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) next.b[j] = cat_bf16(blo[j], bhi[j]);
  };
  // Opening step t+1: this wave's loads of step t+1 have landed (at most
  // `ahead` later stages of 4 loads each remain in flight) and so have its
  // reads of stage t; after the barrier every wave is past that point, so
  // stage t's buffer is refilled with step t + NS when one remains.
  auto open_step = [&](int ahead, bool refill, uint64_t next_step, int buf) {
    if (ahead >= 2) {
      CATENA_WAIT_VMCNT(8);
    } else if (ahead == 1) {
      CATENA_WAIT_VMCNT(4);
    } else {
      CATENA_WAIT_VMCNT(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (refill) issue(next_step, buf);
  };

  // Host guarantees nk = K / 32 is even and nk >= NS.
  static_assert(NS == 4, "the unrolled tail below assumes four stages");
  const uint64_t nk = K / BK;
#pragma unroll
  for (int st = 0; st < NS; ++st) issue(st, st);
  CATENA_WAIT_VMCNT(4 * (NS - 1));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");

  Frags f0, f1;
  load_frags(0, f0);
  // steady state: steps t = 0 .. nk-NS-1 open t+1 and refill with t+NS
  int buf = 0;  // stage of step t
  for (uint64_t t = 0; t < nk - NS; t += 2) {
    const int b1 = buf + 1 == NS ? 0 : buf + 1;
    const int b2 = b1 + 1 == NS ? 0 : b1 + 1;
    open_step(NS - 2, true, t + NS, buf);
    load_mma(b1, f1, f0);
    open_step(NS - 2, true, t + 1 + NS, b1);
    load_mma(b2, f0, f1);
    buf = b2;
  }
  // tail: the last NS steps, nothing left to issue (NS == 4)
  {
    const int b1 = buf + 1 == NS ? 0 : buf + 1;
    const int b2 = b1 + 1 == NS ? 0 : b1 + 1;
    const int b3 = b2 + 1 == NS ? 0 : b2 + 1;
    open_step(2, false, 0, 0);
    load_mma(b1, f1, f0);
    open_step(1, false, 0, 0);
    load_mma(b2, f0, f1);
    open_step(0, false, 0, 0);
    load_mma(b3, f1, f0);
    mma(f1);
  }

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

#define CATENA_GEMM_DEEP_KERNEL(NAME, OUTB, NS, FRONT)                                    \
  extern "C" __global__ __launch_bounds__(512) void NAME(                                 \
      const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, \
      uint64_t M, uint64_t N, uint64_t K) {                                               \
    gemm_deep_body<OUTB, NS, FRONT>(A, B, C, M, N, K);                                    \
  }

CATENA_GEMM_DEEP_KERNEL(catena_gemm_bf16_deep4_bf16out, true, 4, false)
CATENA_GEMM_DEEP_KERNEL(catena_gemm_bf16_deep4_f32out, false, 4, false)
CATENA_GEMM_DEEP_KERNEL(catena_gemm_bf16_deep4f_bf16out, true, 4, true)
CATENA_GEMM_DEEP_KERNEL(catena_gemm_bf16_deep4f_f32out, false, 4, true)
