// bf16 GEMM, aligned shapes (M % 256 == 0, N % BN == 0, K % 128 == 0): the
// default tile kernels.  Four 32-k stages in LDS fed by buffer loads spread
// through the MFMA stream, and (bf16 output) an LDS-staged epilogue that
// writes whole 128-byte rows.
//
// Contraction, tile and order are those of gemm_bf16_lds.hip (reference
// semantics: catena-lang/stdlib/matrix.hex:236-327 on bf16 inputs widened
// exactly, f32 accumulation, NN row-major): one workgroup per 256 x BN
// output tile, v_mfma_f32_16x16x32_bf16 with the B fragment as the first
// operand, K ascending in k32 steps, no split-K, no atomics, so the output
// is bitwise identical to the other tile kernels and run to run (each
// output element sees the same MFMA sequence whatever the tile width).
//
// Tile widths (8 waves each):
//   BN = 256: waves 2 (m) x 4 (n), wave tile 128 x 64 (8 x 4 MFMA blocks);
//   BN = 128: waves 4 (m) x 2 (n), wave tile  64 x 64 (4 x 4 MFMA blocks),
//     for shapes whose 256 x 256 tiles leave CUs idle (the host picks).
//
// Pipeline (S = 4 stages of A [256][32] + B [32][BN]):
//   step s multiplies slab s (fragments already in registers), reads slab
//   s+1's fragments from its stage between its first MFMAs (one read per
//   MFMA), and issues slab s+4 into slab s's stage (free since the barrier
//   that closed step s-1), the loads spread over the step.  The barrier that
//   closes step s waits for slab s+2 only, so a slab has about three steps
//   to arrive.  Slabs past the end are loaded through descriptors with no
//   records: the hardware returns zeros without touching memory, and every
//   step keeps the same wait counts.
//   Spreading the loads matters: the CU's global->LDS path moves 64 B per
//   clock, half of what the MFMAs consume in a step (BN = 256), and a burst
//   of loads at the barrier stalls the issuing waves.
// LDS layout: A stages [S][256][32] then B stages [S][32][BN], so every read
// offset from the per-lane bases fits a DS instruction's immediate.
// Swizzles (conflict-free through the direct-to-LDS write layout):
//   A [256][64 B]:   LDS chunk p of row r holds global chunk p ^ ((r >> 1) & 3).
//                    Measured with SQ_LDS_BANK_CONFLICT on gfx950, the
//                    fragment read (lane 16 G + s: row s, chunk G) costs 8
//                    LDS cycles per ds_read_b128 with p ^ ((r >> 2) & 3) or
//                    no swizzle and the conflict-free 4 with this one;
//   B [32][2*BN B]:  LDS chunk p of row k holds global chunk p ^ hB(k),
//                    hB(k) = 2 * ((k & 3) | ((k >> 3) & 1) << 2)  (row bit 4
//                    unused, so a load 16 rows further shares the lane offset).
#include <type_traits>

#include "common.h"

namespace {
constexpr int BM = 256, BK = 32, S = 4;
constexpr int A_ST = BM * BK;  // elements per A stage
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

CATENA_DEV uint32_t hB(uint32_t k) { return 2u * ((k & 3u) | (((k >> 3) & 1u) << 2)); }

CATENA_DEV bf16x8_t cat_bf16(i16x4_t lo, i16x4_t hi) {
  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  i16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_t, v);
}

// Tile order: consecutive workgroup ids go to different XCDs (round-robin
// dispatch), and each XCD's share is walked in groups of 4 tile rows so its
// L2 holds the A rows and B columns that neighbouring workgroups reuse.
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

// buffer descriptor word 3 for raw (unswizzled, stride 0) 32-bit access
constexpr int kRsrcWord3 = 0x00020000;

// The RoPE epilogue's operands (a fused q / k / v projection, one head per
// 128-column tile): the rotation table [positions][64][2] (cos, sin), the
// per-sequence lengths, q [M][H * 128] and the caches [B][H][L][128], bf16.
struct RopeQkv {
  const float* tab;
  const uint32_t* lens;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
  uint32_t Tq, H, L;
};

// K is the depth this workgroup folds; lda (0: K) is A's row stride, which a
// k-split launch sets to the whole depth (A and B then start at the split's
// first k).
template <bool OUT_BF16, int BN, bool SILU = false, bool ROPE = false>
CATENA_DEV void gemm_k32_body(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                              void* __restrict__ C, uint64_t M, uint64_t N, uint64_t K,
                              const RopeQkv& rq = RopeQkv{}, uint64_t lda = 0) {
  const uint64_t LDA = lda ? lda : K;
  static_assert(!ROPE || BN == 128, "the RoPE epilogue pairs the two column waves of a 128-wide tile");
  static_assert(BN == 256 || BN == 128, "tile widths 256 and 128");
  constexpr int B_ST = BK * BN;                // elements per B stage
  constexpr int WI = BN == 256 ? 8 : 4;        // 16-row MFMA blocks per wave
  constexpr int WAVES_N = BN == 256 ? 4 : 2;   // waves across the tile's columns
  constexpr int NB_LOADS = BN / 128;           // B loads per wave per slab
  constexpr int LOADS = 2 + NB_LOADS;          // loads per wave per slab
  constexpr int READS = WI + 8;                // fragment reads per wave per step
  constexpr int MFMAS = WI * 4;                // MFMAs per wave per step
  constexpr int B_LANES = BN / 8;              // lanes per B row in one load
  extern __shared__ __attribute__((aligned(1024))) uint16_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform, 0..7
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const uint32_t tiles_m = (uint32_t)(M / BM), tiles_n = (uint32_t)(N / BN);
  uint32_t tm, tn;
  tile_of(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const uint64_t m0 = (uint64_t)tm * BM, n0 = (uint64_t)tn * BN;

  // Loads per slab: A 16 one-KiB instructions (16 rows of 64 B each) and B
  // BN / 16 (64 / B_LANES rows of 2 * BN bytes each); per wave 2 of A, the
  // second 16 rows below the first, and NB_LOADS of B, the second 16 rows
  // below the first (soffset), with the lane offsets of the first.
  uint32_t aoff, boff;
  {
    const uint32_t r = 32 * wave + (lane >> 2);
    const uint32_t q = (uint32_t)(lane & 3) ^ ((r >> 1) & 3u);
    aoff = (uint32_t)((r * LDA + 8 * q) * 2);
    const uint32_t kr = (64 / B_LANES) * wave + (uint32_t)lane / B_LANES;
    const uint32_t qb = (uint32_t)(lane % B_LANES) ^ hB(kr);
    boff = (uint32_t)((kr * N + 8 * qb) * 2);
  }
  // Load idx (0, 1: A; 2 .. LOADS-1: B) of slab `slab` into stage `stage`.
  auto issue_one = [&](uint64_t slab, int stage, int idx) {
    const uint64_t k0 = slab * BK;
    const bool live = k0 < K;
    if (idx < 2) {
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(A + m0 * LDA + (live ? k0 : 0)), (short)0, live ? (int)(BM * LDA * 2) : 0, kRsrcWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void*)(smem + stage * A_ST + (32 * wave + 16 * idx) * BK), 16, (int)aoff,
          idx ? (int)(16 * LDA * 2) : 0, 0, 0);
    } else {
      const int b = idx - 2;
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(B + (live ? k0 : 0) * N + n0), (short)0, live ? (int)(BK * N * 2) : 0, kRsrcWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rs, (lds_void*)(smem + S * A_ST + stage * B_ST + ((64 / B_LANES) * wave + 16 * b) * BN), 16,
          (int)boff, b ? (int)(16 * N * 2) : 0, 0, 0);
    }
  };

  // RoPE epilogue: this wave's rotation values (its half of the pair's rows,
  // its 16 columns per col block), requested now so they land during the
  // main loop.  Row blocks (wn * WI / 2 + ii) of the wave's 64 rows.
  f32x4_t rcs[ROPE ? WI : 1][2][2];
  uint32_t rsect = 0;
  if constexpr (ROPE) {
    const int G_ = lane >> 4, s_ = lane & 15;
    rsect = (uint32_t)(n0 / 128) / rq.H;
    if (rsect != 2) {
#pragma unroll
      for (int i = 0; i < WI; ++i) {
        const uint64_t gr = m0 + wm * 64 + 16 * i + s_;
        const uint32_t b = (uint32_t)(gr / rq.Tq), tq = (uint32_t)(gr % rq.Tq);
        const uint32_t len = rq.lens[b];
        const bool ok = len >= rq.Tq && len - rq.Tq + tq < rq.L;
        const uint32_t pos = ok ? len - rq.Tq + tq : 0u;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const f32x4_t* cs =
              reinterpret_cast<const f32x4_t*>(rq.tab + ((uint64_t)pos * 64 + 32 * wn + 16 * j + 4 * G_) * 2);
          rcs[i][j][0] = cs[0];
          rcs[i][j][1] = cs[1];
        }
      }
    }
  }

  f32x4_t acc[WI][4];  // [row block i][col block j], transposed blocks
#pragma unroll
  for (int i = 0; i < WI; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Fragment read bases.  A: lane (G, s) reads row wm*16*WI + 16 i + s, chunk
  // G ^ ((s >> 1) & 3) (row + 16 i leaves the swizzle unchanged).  B: two
  // ds_read_b64_tr_b16 per 32x16 block (rows 8G + s/4 and +4, columns
  // 16 j + 4 (s % 4)), so lane i of a 16-lane group receives 4 consecutive k
  // of one column, matching A's k order.
  const int G = lane >> 4, s = lane & 15;
  auto wave_col = [&](int j) -> uint32_t {
    return ROPE ? (uint32_t)((j >> 1) * 64 + wn * 32 + 16 * (j & 1)) : (uint32_t)(wn * 64 + 16 * j);
  };
  const uint32_t a_lds = (wm * 16 * WI + s) * BK * 2 + 16 * ((uint32_t)G ^ ((uint32_t)(s >> 1) & 3u));
  const uint32_t b_krow = 8 * G + (s >> 2);
  const uint32_t hb = hB(b_krow);
  uint32_t b_lds[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    // col block j of the wave: 16 columns from wave_col(j); the RoPE
    // instance gives wave wn columns 32 wn .. +31 and 64 + 32 wn .. +31, so
    // that each wave holds both members (i, i + 64) of its rotation pairs
    const uint32_t col = wave_col(j) + 4 * (s & 3);
    b_lds[j] = S * A_ST * 2 + b_krow * BN * 2 + 16 * ((col >> 3) ^ hb) + 2 * (col & 7);
  }

  struct Frags {
    bf16x8_t a[WI];
    bf16x8_t b[4];
  };
  auto load_frags = [&](int stage, Frags& f) {
    const char* sa = reinterpret_cast<const char*>(smem + stage * A_ST);
    const char* sb = reinterpret_cast<const char*>(smem + stage * B_ST);
#pragma unroll
    for (int i = 0; i < WI; ++i)
      f.a[i] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(sa + a_lds + i * 16 * BK * 2));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + b_lds[j]));
      i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + b_lds[j] + 4 * BN * 2));
      f.b[j] = cat_bf16(lo, hi);
    }
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int i = 0; i < WI; ++i)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
  };
  // One step: the MFMAs of `cur`; the reads of `next` from stage rs one per
  // MFMA over the first READS; slab islab's LOADS loads into stage ws spread
  // over the step (after MFMA LOAD_AT(l)).  Scheduling barriers pin the
  // interleave, one group per scheduling region.
  // Wave priority falls 3 -> 2 -> 1 -> 0 over the four quarters of the
  // step's MFMAs, so whichever of a SIMD's two waves is ahead yields the
  // issue slot to the one behind.  Without it the older wave (the hardware
  // breaks ties by age) finishes its MFMAs early and the younger one issues
  // the rest alone, at about one MFMA per 27 cycles instead of 16
  // (in-kernel timestamps: 767 against 1,200 cycles per step, then a long
  // barrier wait); measured 2-4% faster on 4096^3.  Each s_setprio closes
  // a scheduling region, so the interleave barriers are emitted per quarter.
  auto load_at = [](int l) { return (l * MFMAS) / LOADS; };
  constexpr int QUARTER = MFMAS / 4;
  auto step = [&](int rs, Frags& next, const Frags& cur, uint64_t islab, int ws) {
    const char* sa = reinterpret_cast<const char*>(smem + rs * A_ST);
    const char* sb = reinterpret_cast<const char*>(smem + rs * B_ST);
    i16x4_t blo[4], bhi[4];
#pragma unroll
    for (int g = 0; g < MFMAS; ++g) {
      if (g == 0) __builtin_amdgcn_s_setprio(3);
      if (g == QUARTER) __builtin_amdgcn_s_setprio(2);
      if (g == 2 * QUARTER) __builtin_amdgcn_s_setprio(1);
      if (g == 3 * QUARTER) __builtin_amdgcn_s_setprio(0);
      if (g < WI) {
        next.a[g] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(sa + a_lds + g * 16 * BK * 2));
      } else if (g < READS) {
        const int j = (g - WI) >> 1;
        if (((g - WI) & 1) == 0)
          blo[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + b_lds[j]));
        else
          bhi[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(sb + b_lds[j] + 4 * BN * 2));
      }
      const int j = g / WI, i = g % WI;
      acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
#pragma unroll
      for (int l = 0; l < LOADS; ++l)
        if (g == load_at(l)) issue_one(islab, ws, l);
      if (g % QUARTER == QUARTER - 1) {
        // this quarter's interleave: one DS read, one MFMA, the loads
#pragma unroll
        for (int h = g - (QUARTER - 1); h <= g; ++h) {
          if (h < READS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
#pragma unroll
          for (int l = 0; l < LOADS; ++l)
            if (h == load_at(l)) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) next.b[j] = cat_bf16(blo[j], bhi[j]);
  };
  // Closing a step: this wave's fragment reads have landed and its loads of
  // slab s+2 have (two later slabs of LOADS loads stay in flight); after the
  // barrier every wave is past the same point.
  auto end_step = [&]() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    CATENA_WAIT_VMCNT(LOADS * (S - 2));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  const uint64_t nk = K / BK;  // host guarantees nk % S == 0
#pragma unroll
  for (int t = 0; t < S; ++t)
#pragma unroll
    for (int q = 0; q < LOADS; ++q) issue_one((uint64_t)t, t, q);
  CATENA_WAIT_VMCNT(LOADS * (S - 2));  // slabs 0 and 1 landed
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  Frags f0, f1;
  load_frags(0, f0);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();  // stage 0 may be refilled
  asm volatile("" ::: "memory");
  for (uint64_t sb = 0; sb < nk; sb += S) {
#pragma unroll
    for (int t = 0; t < S; t += 2) {
      step((t + 1) % S, f1, f0, sb + t + S, t);
      end_step();
      step((t + 2) % S, f0, f1, sb + t + 1 + S, t + 1);
      end_step();
    }
  }
  CATENA_WAIT_VMCNT(0);  // no LDS writes outstanding past this point

  if constexpr (SILU) {
    // SwiGLU: B's columns come in groups of 64, gate and up alternating (a
    // 128-column group holds matching gate and up columns), so a wave with
    // even wn holds gate columns and wave wn + 1 the matching up columns.
    // C is act [M][N / 2]: act[m][(n0 + 64 (wn & ~1)) / 2 + c] =
    // bf16(silu~(gate) * up) of the f32 tile, as catena_silu_mul_bf16 with
    // group 64.  Both waves of a pair work: the gate wave takes the first
    // half of the rows, the up wave the second, each handing the other the
    // half it needs through LDS (rows skewed by 16 bytes), so every SIMD
    // carries two waves of the SiLU arithmetic.  Each wave then stages its
    // act rows like the bf16 tile below and stores whole 128-byte rows.
    constexpr int UP_LD = 68;                 // f32 row stride of a pair's slot
    constexpr int SLOT = WI * 16 * UP_LD;     // floats per slot
    constexpr int HB = WI / 2;                // row blocks per wave
    float* slot = reinterpret_cast<float*>(smem) + (wm * (WAVES_N / 2) + (wn >> 1)) * SLOT;
    const int half = wn & 1;                  // 0: gate wave, first rows; 1: up wave, last rows
    // Each phase is instantiated for both halves so every acc index is a
    // compile-time constant (a run-time index would put acc in scratch).
    auto hand_over = [&](auto H) {
      constexpr int h = decltype(H)::value;
#pragma unroll
      for (int ii = 0; ii < HB; ++ii) {
        constexpr int base = (1 - h) * HB;    // the partner's row blocks
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<f32x4_t*>(slot + (16 * (base + ii) + s) * UP_LD + 16 * j + 4 * G) = acc[base + ii][j];
      }
    };
    if (half)
      hand_over(std::integral_constant<int, 1>{});
    else
      hand_over(std::integral_constant<int, 0>{});
    __syncthreads();
    uint2 act[HB][4];
    auto swiglu = [&](auto H) {
      constexpr int h = decltype(H)::value;
#pragma unroll
      for (int ii = 0; ii < HB; ++ii) {
        constexpr int base = h * HB;          // this wave's row blocks
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4_t other =
              *reinterpret_cast<const f32x4_t*>(slot + (16 * (base + ii) + s) * UP_LD + 16 * j + 4 * G);
          float a[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gate = h ? other[q] : acc[base + ii][j][q];
            const float up = h ? acc[base + ii][j][q] : other[q];
            const float sg = silu_approx(gate);
            a[q] = sg * up;
          }
          act[ii][j].x = pack_bf16x2(a[0], a[1]);
          act[ii][j].y = pack_bf16x2(a[2], a[3]);
        }
      }
    };
    if (half)
      swiglu(std::integral_constant<int, 1>{});
    else
      swiglu(std::integral_constant<int, 0>{});
    __syncthreads();  // the slots are read; every wave stages below
    char* wt = reinterpret_cast<char*>(smem) + wave * (HB * 16 * 128);
#pragma unroll
    for (int ii = 0; ii < HB; ++ii) {
      const uint32_t r = 16 * ii + s;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = (uint32_t)(2 * j + (G >> 1)) ^ ((r >> 1) & 7u);
        *reinterpret_cast<uint2*>(wt + r * 128 + 16 * c + 8 * (G & 1)) = act[ii][j];
      }
    }
    const uint64_t F = N / 2;
    const uint32_t rr = (uint32_t)lane >> 3, cc = (uint32_t)lane & 7;
#pragma unroll
    for (int t = 0; t < WI; ++t) {
      const uint32_t r = 8 * t + rr;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wt + r * 128 + 16 * (cc ^ ((r >> 1) & 7u)));
      const uint64_t gr = m0 + wm * 16 * WI + half * HB * 16 + r;
      const uint64_t gc = (n0 + (wn & ~1) * 64) / 2 + 8 * cc;
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(C) + gr * F + gc) = v;
    }
  } else if constexpr (ROPE) {
    // RoPE + bf16 + cache append (catena_rope_qkv_store's arithmetic, the
    // rotation read from the table the same functions built, requested
    // before the main loop).  The tile is one head: section n0 / 128 / H
    // (0 q, 1 k, 2 v), head n0 / 128 % H.  Col blocks 0, 1 of a wave hold x1
    // of pairs i = 32 wn + 16 j + .., blocks 2, 3 the matching x2 (columns
    // i + 64), so every lane rotates its own values:
    //   y1 = x1 c - x2 s, y2 = x2 c + x1 s (q and k; v unrotated), each op
    //   rounded, c / s at the row's position pos = lens[b] - Tq + tq.
    // Each wave stages its 64 rows x (32 + 32) bf16 (row r, 16-byte chunk c
    // at r * 128 + 16 (c ^ ((r >> 1) & 7)); chunks 0-3 the y1 columns, 4-7
    // the y2 columns) and stores 64-byte runs: q rows always, cache rows when
    // pos < L (a row before the cache start reads the table at position 0
    // and writes q only).  No barrier: each wave uses its own LDS.
    const uint32_t hcol = (uint32_t)(n0 / 128);
    const uint32_t sect = rsect, head = hcol % rq.H;
    char* wt = reinterpret_cast<char*>(smem) + wave * (WI * 16 * 128);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const uint32_t r = 16 * i + s;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f32x4_t x1 = acc[i][j], x2 = acc[i][j + 2];
        f32x4_t y1, y2;
        if (sect == 2) {
          y1 = x1;
          y2 = x2;
        } else {
          const f32x4_t cs0 = rcs[i][j][0], cs1 = rcs[i][j][1];  // (c, s) of pairs i .. i + 3
          const float cv[4] = {cs0[0], cs0[2], cs1[0], cs1[2]};
          const float sv[4] = {cs0[1], cs0[3], cs1[1], cs1[3]};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float t1 = x1[q] * cv[q], t2 = x2[q] * sv[q], t3 = x2[q] * cv[q], t4 = x1[q] * sv[q];
            y1[q] = t1 - t2;
            y2[q] = t3 + t4;
          }
        }
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const f32x4_t yv = w ? y2 : y1;
          uint2 p;
          p.x = pack_bf16x2(yv[0], yv[1]);
          p.y = pack_bf16x2(yv[2], yv[3]);
          const uint32_t c = (uint32_t)(4 * w + 2 * j + (G >> 1)) ^ ((r >> 1) & 7u);
          *reinterpret_cast<uint2*>(wt + r * 128 + 16 * c + 8 * (G & 1)) = p;
        }
      }
    }
    const uint64_t HD = (uint64_t)rq.H * 128;
#pragma unroll
    for (int t = 0; t < WI * 2; ++t) {
      const uint32_t idx = 64 * t + lane;
      const uint32_t r = idx >> 3, c = idx & 7;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wt + r * 128 + 16 * (c ^ ((r >> 1) & 7u)));
      const uint64_t gr = m0 + wm * 64 + r;
      const uint32_t col = (c >> 2) * 64 + wn * 32 + 8 * (c & 3);
      const uint32_t b = (uint32_t)(gr / rq.Tq), tq = (uint32_t)(gr % rq.Tq);
      const uint32_t len = rq.lens[b];
      const bool ok = len >= rq.Tq && len - rq.Tq + tq < rq.L;
      if (sect == 0) {
        *reinterpret_cast<u32x4_t*>(rq.q_out + gr * HD + (uint64_t)head * 128 + col) = v;
      } else if (ok) {
        const uint32_t pos = len - rq.Tq + tq;
        uint16_t* cache = sect == 1 ? rq.kc : rq.vc;
        *reinterpret_cast<u32x4_t*>(cache + (((uint64_t)b * rq.H + head) * rq.L + pos) * 128 + col) = v;
      }
    }
  } else if constexpr (OUT_BF16) {
    // Stage the wave's (16 WI) x 64 bf16 tile in its own LDS (row r, 16-byte
    // chunk c at r * 128 + 16 * (c ^ ((r >> 1) & 7))), then store whole
    // 128-byte rows: 8 lanes per row, 8 rows per instruction.  The barrier
    // above (closing the last step) left every wave done with the stages.
    char* wt = reinterpret_cast<char*>(smem) + wave * (WI * 16 * 128);
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const uint32_t r = 16 * i + s;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4_t v = acc[i][j];
        uint2 p;
        p.x = pack_bf16x2(v[0], v[1]);
        p.y = pack_bf16x2(v[2], v[3]);
        const uint32_t c = (uint32_t)(2 * j + (G >> 1)) ^ ((r >> 1) & 7u);
        *reinterpret_cast<uint2*>(wt + r * 128 + 16 * c + 8 * (G & 1)) = p;
      }
    }
    const uint32_t rr = (uint32_t)lane >> 3, cc = (uint32_t)lane & 7;
#pragma unroll
    for (int t = 0; t < 2 * WI; ++t) {
      const uint32_t r = 8 * t + rr;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wt + r * 128 + 16 * (cc ^ ((r >> 1) & 7u)));
      const uint64_t gr = m0 + wm * 16 * WI + r;
      const uint64_t gc = n0 + wn * 64 + 8 * cc;
      *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(C) + gr * N + gc) = v;
    }
  } else {
    // acc[i][j] lane (G, s) holds C[row 16 i + s][cols 16 j + 4G .. +3]
#pragma unroll
    for (int i = 0; i < WI; ++i) {
      const uint64_t gr = m0 + wm * 16 * WI + 16 * i + s;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint64_t gc = n0 + wn * 64 + 16 * j + 4 * G;
        *reinterpret_cast<f32x4_t*>(static_cast<float*>(C) + gr * N + gc) = acc[i][j];
      }
    }
  }
}
}  // namespace

#define CATENA_GEMM_K32_KERNEL(NAME, OUTB, BN_)                                           \
  extern "C" __global__ __launch_bounds__(512) void NAME(                                 \
      const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, \
      uint64_t M, uint64_t N, uint64_t K) {                                               \
    gemm_k32_body<OUTB, BN_>(A, B, C, M, N, K);                                           \
  }

// grid = (M / 256) * (N / BN), block = 512, dynamic LDS S * (256 + BN) * 32 * 2 B
CATENA_GEMM_K32_KERNEL(catena_gemm_bf16_k32_bf16out, true, 256)
CATENA_GEMM_K32_KERNEL(catena_gemm_bf16_k32_f32out, false, 256)
CATENA_GEMM_K32_KERNEL(catena_gemm_bf16_k32n128_bf16out, true, 128)
CATENA_GEMM_K32_KERNEL(catena_gemm_bf16_k32n128_f32out, false, 128)

// SwiGLU-fused: C = act [M][N / 2] bf16 (N % 128 == 0), dynamic LDS the larger
// of the stages and 4 up slots of 16 WI rows x 68 floats
#define CATENA_GEMM_K32_SILU_KERNEL(NAME, BN_)                                            \
  extern "C" __global__ __launch_bounds__(512) void NAME(                                 \
      const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, void* __restrict__ C, \
      uint64_t M, uint64_t N, uint64_t K) {                                               \
    gemm_k32_body<false, BN_, true>(A, B, C, M, N, K);                                    \
  }
CATENA_GEMM_K32_SILU_KERNEL(catena_gemm_bf16_k32_silu, 256)
CATENA_GEMM_K32_SILU_KERNEL(catena_gemm_bf16_k32n128_silu, 128)

// RoPE + cache append fused (256 x 128 tiles, one head each): no C output;
// q_out [M][H * 128], kc / vc [B][H][L][128] bf16 (N = 3 H 128, M = B Tq).
// Dynamic LDS: the stages (96 KiB), which cover the 8 waves' 64 x 128-byte
// staging.
extern "C" __global__ __launch_bounds__(512) void catena_gemm_bf16_k32n128_rope(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, uint64_t M, uint64_t N,
    uint64_t K, const float* __restrict__ tab, const uint32_t* __restrict__ lens,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    uint32_t Tq, uint32_t H, uint32_t L) {
  const RopeQkv rq{tab, lens, q_out, kc, vc, Tq, H, L};
  gemm_k32_body<false, 128, false, true>(A, B, nullptr, M, N, K, rq);
}

// k-split f32 partials (256 x 256 tiles): grid (tiles, splits); split z folds
// k in [z k_len, (z + 1) k_len) of the K_total-deep product in the tile
// kernel's order and writes P[z] = its [M][N] f32 partial.  The consumer adds
// P[0] + P[1] + ... in ascending z.  Dynamic LDS as the 256 x 256 kernel.
extern "C" __global__ __launch_bounds__(512) void catena_gemm_bf16_k32_f32parts(
    const uint16_t* __restrict__ A, const uint16_t* __restrict__ B, float* __restrict__ P,
    uint64_t M, uint64_t N, uint64_t K_total, uint64_t k_len) {
  const uint64_t z = blockIdx.y;
  gemm_k32_body<false, 256>(A + z * k_len, B + z * k_len * N, P + z * M * N, M, N, k_len, RopeQkv{},
                            K_total);
}
