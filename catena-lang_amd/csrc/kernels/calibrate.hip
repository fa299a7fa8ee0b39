// Measurement kernels for bench.py's ceilings (not part of the library's
// path: the host library never loads this code object).  Each one isolates
// one resource the hot kernels are bound by, on the data the bench uses:
//
//   catena_calib_mfma_bf16      16x16x32 bf16 MFMAs only, random operands in
//                               registers (the MFMA power draw, and so the
//                               clock, depends on the operand bits).
//   catena_calib_mfma_lds_bf16  the same MFMAs fed from LDS at the bf16 GEMM's
//                               ratio (per 32 MFMAs 8 ds_read_b128 + 8
//                               ds_read_b64, two fragment sets alternating).
//   catena_calib_mfma_lds_4w_bf16  the same LDS-fed loop shaped for one
//                               wave per SIMD with a 128 x 128 wave tile: 64
//                               MFMAs per step against 8 ds_read_b128 + 16
//                               ds_read_b64 (a third fewer LDS bytes per
//                               MFMA), the 256 accumulator registers in AGPRs.
//   catena_calib_read           plain HBM read, one contiguous chunk per
//                               workgroup, four 16-byte loads in flight.
//   catena_calib_read_nt        the same with non-temporal loads.
//   catena_calib_write_tile     the 4096^2 bf16 GEMM's C store: 256 x 256
//                               tiles, 128-byte rows, all workgroups at once.
//
// The MFMA kernels write, per wave, the s_memtime (shader clock) and
// s_memrealtime (100 MHz) deltas of their timed loop to cyc[2 w], cyc[2 w + 1].
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

__device__ inline uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
// A finite bf16 with random sign and mantissa and exponent 126..128 (|x| in
// [0.5, 4)): the bit activity of N(0, 1) data without overflow over long
// accumulations.
__device__ inline uint32_t rand_bf16(uint32_t h) {
  return ((h & 1u) << 15) | ((126u + (h >> 1) % 3u) << 7) | ((h >> 8) & 0x7fu);
}

__device__ inline void stamp(uint64_t& clk, uint64_t& real) {
  asm volatile("s_memtime %0\n s_memrealtime %1\n s_waitcnt lgkmcnt(0)" : "=s"(clk), "=s"(real));
}

__device__ inline void write_cycles(uint64_t* cyc, uint64_t c0, uint64_t r0, uint64_t c1, uint64_t r1) {
  if ((threadIdx.x & 63) == 0) {
    const uint32_t w = blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    cyc[2 * w] = c1 - c0;
    cyc[2 * w + 1] = r1 - r0;
  }
}

struct LdsFrags {
  bf16x8_t a[8];
  bf16x8_t b[4];
};

// 32 MFMAs of `cur` with the reads of `nx` (from p) interleaved one per MFMA.
__device__ inline void lds_half_step(f32x4_t (&acc)[32], LdsFrags& nx, const LdsFrags& cur, const char* p) {
  u32x2_t lo[4], hi[4];
#pragma unroll
  for (int g = 0; g < 32; ++g) {
    if (g < 8) {
      nx.a[g] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(p + g * 1024));
    } else if (g < 16) {
      const int j = (g - 8) >> 1;
      if ((g & 1) == 0)
        lo[j] = *reinterpret_cast<const u32x2_t*>(p + 8192 + j * 1024);
      else
        hi[j] = *reinterpret_cast<const u32x2_t*>(p + 8192 + j * 1024 + 512);
    }
    acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[g >> 3], cur.a[g & 7], acc[g], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x4_t v = {lo[j][0], lo[j][1], hi[j][0], hi[j][1]};
    nx.b[j] = __builtin_bit_cast(bf16x8_t, v);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
}

}  // namespace

// grid any, block 512; out[grid * 512], cyc[2 * grid * 8].  iters MFMAs x 32 per wave.
extern "C" __global__ __launch_bounds__(512) void catena_calib_mfma_bf16(float* out, uint64_t* cyc, int iters,
                                                                          uint32_t seed) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  f32x4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bf16x8_t a[4], b[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    i16x8_t ra, rb;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = mix32((tid * 64 + p * 16 + e) ^ seed);
      ra[e] = (short)rand_bf16(h);
      rb[e] = (short)rand_bf16(h >> 16 | h << 16);
    }
    a[p] = __builtin_bit_cast(bf16x8_t, ra);
    b[p] = __builtin_bit_cast(bf16x8_t, rb);
  }
  __syncthreads();
  uint64_t c0, r0, c1, r1;
  stamp(c0, r0);
#pragma unroll
  for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(acc[i]));
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 32; ++i)
      acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i & 3], b[(i >> 2) & 3], acc[i], 0, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(acc[i]));
  stamp(c1, r1);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) s += acc[i][0] + acc[i][3];
  out[tid] = s;
  write_cycles(cyc, c0, r0, c1, r1);
}

// grid any, block 512, 64 KiB static LDS; out[grid * 512], cyc[2 * grid * 8];
// iters even, 32 MFMAs per iteration per wave.
extern "C" __global__ __launch_bounds__(512) void catena_calib_mfma_lds_bf16(float* out, uint64_t* cyc, int iters,
                                                                              uint32_t seed) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[16384];
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  for (uint32_t i = threadIdx.x; i < 16384; i += blockDim.x) {
    const uint32_t h = mix32((tid * 131 + i) ^ seed), g = mix32(h);
    lds[i] = rand_bf16(h) | (rand_bf16(g) << 16);
  }
  f32x4_t acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  // Byte offsets read: 16 * lane (<= 1008) plus at most 32768 + 8192 + 3 * 1024
  // + 512 + 8 bytes: 45,560 < 65,536.
  const char* base = reinterpret_cast<const char*>(lds) + 16 * (threadIdx.x & 63);
  LdsFrags f0, f1;
#pragma unroll
  for (int p = 0; p < 8; ++p) f0.a[p] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(base + p * 1024));
#pragma unroll
  for (int p = 0; p < 4; ++p)
    f0.b[p] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(base + 8192 + p * 1024));
  __builtin_amdgcn_s_waitcnt(0xC07F);
  uint64_t c0, r0, c1, r1;
  stamp(c0, r0);
#pragma unroll
  for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(acc[i]));
  for (int it = 0; it < iters; it += 2) {
    lds_half_step(acc, f1, f0, base + 16384);
    lds_half_step(acc, f0, f1, base + 32768);
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) asm volatile("" : "+v"(acc[i]));
  stamp(c1, r1);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) s += acc[i][0] + acc[i][3];
  out[tid] = s;
  write_cycles(cyc, c0, r0, c1, r1);
}

namespace {
struct LdsFrags8 {
  bf16x8_t a[8];
  bf16x8_t b[8];
};

// 64 MFMAs of `cur` (8 x 8 blocks) with the 24 reads of `nx` (from p)
// interleaved one per MFMA.
__device__ inline void lds_step64(f32x4_t (&acc)[64], LdsFrags8& nx, const LdsFrags8& cur, const char* p) {
  u32x2_t lo[8], hi[8];
#pragma unroll
  for (int g = 0; g < 64; ++g) {
    if (g < 8) {
      nx.a[g] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(p + g * 1024));
    } else if (g < 24) {
      const int j = (g - 8) >> 1;
      if ((g & 1) == 0)
        lo[j] = *reinterpret_cast<const u32x2_t*>(p + 8192 + j * 1024);
      else
        hi[j] = *reinterpret_cast<const u32x2_t*>(p + 8192 + j * 1024 + 512);
    }
    acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.b[g >> 3], cur.a[g & 7], acc[g], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const u32x4_t v = {lo[j][0], lo[j][1], hi[j][0], hi[j][1]};
    nx.b[j] = __builtin_bit_cast(bf16x8_t, v);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
}
}  // namespace

// grid any, block 256 (one wave per SIMD), 64 KiB static LDS; out[grid * 256],
// cyc[2 * grid * 4]; iters even, 64 MFMAs per iteration per wave.
extern "C" __global__ __launch_bounds__(256, 1) void catena_calib_mfma_lds_4w_bf16(float* out, uint64_t* cyc,
                                                                                   int iters, uint32_t seed) {
  __shared__ __attribute__((aligned(16))) uint32_t lds[16384];
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  for (uint32_t i = threadIdx.x; i < 16384; i += blockDim.x) {
    const uint32_t h = mix32((tid * 131 + i) ^ seed), g = mix32(h);
    lds[i] = rand_bf16(h) | (rand_bf16(g) << 16);
  }
  f32x4_t acc[64];
#pragma unroll
  for (int i = 0; i < 64; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  __syncthreads();
  // Byte offsets read: 16 * lane (<= 1008) plus at most 32768 + 8192 + 7 * 1024
  // + 512 + 8 bytes: 49,656 < 65,536.
  const char* base = reinterpret_cast<const char*>(lds) + 16 * (threadIdx.x & 63);
  LdsFrags8 f0, f1;
#pragma unroll
  for (int p = 0; p < 8; ++p) f0.a[p] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(base + p * 1024));
#pragma unroll
  for (int p = 0; p < 8; ++p)
    f0.b[p] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t*>(base + 8192 + p * 1024));
  __builtin_amdgcn_s_waitcnt(0xC07F);
  uint64_t c0, r0, c1, r1;
  stamp(c0, r0);
  for (int it = 0; it < iters; it += 2) {
    lds_step64(acc, f1, f0, base + 16384);
    lds_step64(acc, f0, f1, base + 32768);
  }
  stamp(c1, r1);
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 64; ++i) s += acc[i][0] + acc[i][3];
  out[tid] = s;
  write_cycles(cyc, c0, r0, c1, r1);
}

// grid G, block 512: workgroup b reads the 16-byte words [b * per_wg, (b + 1) *
// per_wg) of src (per_wg a multiple of 2048); flag[0] is written only if the
// xor of everything read equals `never` (keeps the loads).
extern "C" __global__ __launch_bounds__(512) void catena_calib_read(const u32x4_t* __restrict__ src, uint64_t per_wg,
                                                                     uint32_t* flag, uint32_t never) {
  u32x4_t acc = {0u, 0u, 0u, 0u};
  const u32x4_t* p = src + (uint64_t)blockIdx.x * per_wg;
  for (uint64_t i = threadIdx.x; i + 1536 < per_wg; i += 2048) {
    const u32x4_t a = p[i], b = p[i + 512], c = p[i + 1024], d = p[i + 1536];
    acc ^= a ^ b ^ c ^ d;
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == never) flag[0] = 1u;
}

// The same read with the non-temporal hint on every 16-byte load (whole
// 128-byte lines per wave instruction): the rate the decode attention's K and
// V streams and the plain decode GEMM's weight stream are built for.
extern "C" __global__ __launch_bounds__(512) void catena_calib_read_nt(const u32x4_t* __restrict__ src,
                                                                        uint64_t per_wg, uint32_t* flag,
                                                                        uint32_t never) {
  u32x4_t acc = {0u, 0u, 0u, 0u};
  const u32x4_t* p = src + (uint64_t)blockIdx.x * per_wg;
  for (uint64_t i = threadIdx.x; i + 1536 < per_wg; i += 2048) {
    const u32x4_t a = __builtin_nontemporal_load(p + i), b = __builtin_nontemporal_load(p + i + 512),
                  c = __builtin_nontemporal_load(p + i + 1024), d = __builtin_nontemporal_load(p + i + 1536);
    acc ^= a ^ b ^ c ^ d;
  }
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == never) flag[0] = 1u;
}

// grid 256, block 512: the 4096 x 4096 bf16 matrix C as 16 x 16 tiles of 256 x
// 256, tile b = (b / 16, b % 16); wave w writes rows (w / 4) * 128 .. +127,
// columns (w % 4) * 64 .. +63 of its tile as 128-byte rows, 8 lanes per row.
extern "C" __global__ __launch_bounds__(512) void catena_calib_write_tile(u32x4_t* __restrict__ c, uint32_t v) {
  const uint32_t tm = blockIdx.x / 16, tn = blockIdx.x % 16;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t wm = wave / 4, wn = wave % 4;
  const u32x4_t val = {v ^ lane, v, v + wave, v};
#pragma unroll
  for (int it = 0; it < 16; ++it) {
    const uint64_t gr = (uint64_t)tm * 256 + wm * 128 + it * 8 + (lane >> 3);
    const uint64_t gc = (uint64_t)tn * 256 + wn * 64 + 8 * (lane & 7);
    c[(gr * 4096 + gc) / 8] = val;
  }
}
