// KV-cache attention over a bf16 cache (decode: one query per sequence;
// causal: its last Tq positions), f32 scores and softmax, bitwise equal to
// the sequential composition of the reference's own pieces:
//   s_t = (fold_{d asc} from +0 of q_d * k_{t,d}) * scale
//         -- f32.matmul.cell-dot order, catena-lang/stdlib/matrix.hex:236-256
//   m   = f32.max-env fold from -inf        (catena-lang/stdlib/sum.hex:73-84)
//   den = f32.add-env fold from +0 of exp~(s_t - m)  (catena-lang/stdlib/nn.hex:93-114)
//   p_t = exp~(s_t - m) / den                (catena-lang/stdlib/nn.hex:75-90)
//   o_d = fold_{t asc} from +0 of p_t * v_{t,d}
// exp~ is math.exp-approx (catena-lang/stdlib/math.hex:148-199).
//
// One workgroup (4 waves) per (batch, query, head); layouts q[B][Tq][H][128],
// k/v[B][H][L][128] (bf16, head-major, one 256-byte row per position),
// lens[B] (positions in the cache per sequence, clamped to L),
// o[B][Tq][H][128] (f32, or bf16 RNE).  The Tq queries of a sequence are
// its last Tq positions (causal): query tq attends to the first
// lens[b] - (Tq - 1 - tq) positions.  Tq = 1 is the decode step.
//
// K pass: each wave takes 32-row blocks (blocks w, w+4, ...).  A block is
// moved in two 64-wide d halves: a coalesced 16-byte-per-lane non-temporal
// buffer load (8 lanes per 128-byte row half, so every request is a whole
// 128-byte line; rows past the sequence read as zeros), a write into the
// wave's private LDS slice, and a read back in which lane l (and l + 32,
// repeating it) owns row l, so every score is one lane's d-ascending chain
// of v_mul_f32 + v_add_f32.  Two register sets keep the next two halves'
// loads in flight while one is folded.
// Softmax: the max is the exact parallel form of the sequential fold (see
// FirstMax in common.h); exp~ is elementwise; the denominator is the one
// truly sequential fold and runs as one lane-to-lane chain in wave 0
// (serial_sum_wave_long); p_t is one correctly rounded division per element.
// V pass: waves 0 and 1 own 64 output columns each (lane = column) and walk
// t ascending through 64-row batches staged in LDS, with the next two
// batches' loads in flight while one is folded; the first batch is requested
// before the softmax phase so HBM stays busy through it.  A full batch is
// read back four rows at a time with the transposing LDS read, p four at a
// time.  Every K and V byte is read from HBM once.
#include "common.h"

namespace {
constexpr int D = 128;
// K stage: per wave [32 rows][128 B] (one d half of a 32-row block);
// 16-byte chunk c of row t sits at position c ^ (t & 7) ^ ((t >> 3) & 1).
// A staging write (8 rows x 128 B) puts its four even rows in banks 0-31 and
// its four odd rows in banks 32-63; a read-back instruction (lane t: chunk c
// of row t) covers all 64 banks with every 16 consecutive rows: both take
// the minimum LDS cycles for their bytes.
constexpr int KSTAGE_ROW = 128;
constexpr int KSTAGE_WAVE = 32 * KSTAGE_ROW;  // 4096 B per wave
constexpr int STAGE_BYTES = 4 * KSTAGE_WAVE;  // 16384 B (V pass uses 2 x 8192)
// Raw buffer descriptor word 3 (stride 0, bounds-checked by byte offset) and
// the non-temporal cache policy of a load.
constexpr int kRsrcWord3 = 0x00020000;
constexpr int kCpolNt = 2;
CATENA_DEV uint32_t kswz(uint32_t row, uint32_t chunk) {
  return 16u * (chunk ^ (row & 7u) ^ ((row >> 3) & 1u));
}

// Wave priority p & 3 for the SQ's issue arbitration.  The workgroups of the
// C4 grid that share a CU are blockIdx.x 256 apart; with one priority for
// all, the oldest wins the memory-issue ties and they finish in dispatch
// order (medians 258, 275, 288, 304 us), so the last CUs end late.  Each
// workgroup's priority therefore rotates with its progress, offset by
// blockIdx.x >> 8 (measured 323 -> 317 us; the same bits).
CATENA_DEV void set_prio(uint32_t p) {
  switch (p & 3u) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
  }
}

CATENA_DEV void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4;

CATENA_DEV int wave_max_i32(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    int o = __shfl_xor(v, off, 64);
    v = o > v ? o : v;
  }
  return v;
}

CATENA_DEV FirstMax wave_first_max(FirstMax a) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    FirstMax b;
    b.v = __shfl_xor(a.v, off, 64);
    b.i = (uint32_t)__shfl_xor((int)a.i, off, 64);
    a = first_max_combine(a, b);
  }
  return a;
}
}  // namespace

// K and V are streamed with the non-temporal hint, always as whole 128-byte
// lines per request: measured on gfx950, a plain read of 2 GiB runs at
// 6.0-6.3 TB/s and a non-temporal one at 7.1-7.3 TB/s, but non-temporal
// reads of 64-byte half lines in consecutive steps fetch the line twice
// (5.2-5.7 TB/s).
template <bool OUT_BF16>
CATENA_DEV void attn_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                          const uint16_t* __restrict__ v, const uint32_t* __restrict__ lens,
                          void* __restrict__ o, uint32_t H, uint32_t L, uint32_t Tq,
                          float scale) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* qf = reinterpret_cast<float*>(smem);                  // [128]
  unsigned char* stage = smem + D * 4;                         // [STAGE_BYTES]
  int* red_i = reinterpret_cast<int*>(smem + D * 4 + STAGE_BYTES);        // [4]
  float* red_v = reinterpret_cast<float*>(red_i + 4);                     // [4]
  uint32_t* red_u = reinterpret_cast<uint32_t*>(red_v + 4);               // [4]
  float* sp = reinterpret_cast<float*>(smem + D * 4 + STAGE_BYTES + 64);  // [L]

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint64_t qi = blockIdx.x;  // (b * Tq + tq) * H + h
  const uint32_t row = (uint32_t)(qi / H), h = (uint32_t)(qi % H);
  const uint32_t b = row / Tq, tq = row % Tq;
  const uint64_t bh = (uint64_t)b * H + h;
  uint32_t len = lens[b];
  if (len > L) len = L;
  const uint32_t later = Tq - 1 - tq;  // queries after this one in the sequence
  len = len > later ? len - later : 0;

  const uint16_t* kb = k + bh * (uint64_t)L * D;
  const uint16_t* vb = v + bh * (uint64_t)L * D;
  if (tid < D) qf[tid] = bf16_to_f32(q[qi * D + tid]);
  __syncthreads();

  // ---------------------------------------------------------------- K pass
  // Blocks of 32 rows, each moved as two 64-wide d halves (32 rows x 128 B:
  // whole lines).  Lane l (and l + 32, which repeats its work) folds row l
  // of the block; the K fold's VALU work is small beside the stream.
  {
    unsigned char* st = stage + wave * KSTAGE_WAVE;
    const uint32_t nblk = (len + 31) / 32;
    // this wave's (block, half) steps, flattened
    const uint32_t my_blocks = nblk > (uint32_t)wave ? (nblk - wave + 3) / 4 : 0;
    const uint32_t steps = my_blocks * 2;
    const int lrow = lane >> 3, lchunk = lane & 7;
    const uint32_t frow = (uint32_t)lane & 31u;
    // the (b, h) slice's first len rows as a bounds-checked buffer: rows past
    // len read as zeros without a branch around the load
    const __amdgpu_buffer_rsrc_t krs =
        __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0, (int)(len * (uint32_t)D * 2u), kRsrcWord3);
    const int kvoff = lrow * D * 2 + lchunk * 16;
    auto gload = [&](uint32_t step, u32x4_t r[4]) {
      const uint32_t blk = wave + 4 * (step >> 1), half = step & 1;
      const int soff = (int)(blk * 32u * D * 2u + half * 128u);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        r[i] = __builtin_amdgcn_raw_buffer_load_b128(krs, kvoff, soff + i * 8 * D * 2, kCpolNt);
    };
    // Two register sets: while half `step` is folded, halves step+1 and
    // step+2 are in flight.  steps is even, so the pair loop is exact.
    u32x4_t ra[4], rb[4];
    if (steps > 0) gload(0, ra);
    if (steps > 1) gload(1, rb);
    float acc = __uint_as_float(0u);
    auto process = [&](uint32_t step, u32x4_t* r) {
      const uint32_t half = step & 1;
      set_prio((uint32_t)(qi >> 8) + (step >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t srow = lrow + 8 * i;
        *reinterpret_cast<u32x4_t*>(st + srow * KSTAGE_ROW + kswz(srow, lchunk)) = r[i];
      }
      wave_sync();
      if (step + 2 < steps) gload(step + 2, r);
      if (half == 0) acc = __uint_as_float(0u);
      const unsigned char* myrow = st + frow * KSTAGE_ROW;
      // two chunks per iteration: the q and K reads of a whole half at once
      // would not fit beside the register sets in flight
#pragma unroll 2
      for (int ch = 0; ch < 8; ++ch) {
        const u32x4_t kv = *reinterpret_cast<const u32x4_t*>(myrow + kswz(frow, ch));
        const f32x4_t q0 = *reinterpret_cast<const f32x4_t*>(qf + half * 64 + ch * 8);
        const f32x4_t q1 = *reinterpret_cast<const f32x4_t*>(qf + half * 64 + ch * 8 + 4);
        float p;
        p = q0[0] * bf16lo(kv[0]); acc = acc + p;
        p = q0[1] * bf16hi(kv[0]); acc = acc + p;
        p = q0[2] * bf16lo(kv[1]); acc = acc + p;
        p = q0[3] * bf16hi(kv[1]); acc = acc + p;
        p = q1[0] * bf16lo(kv[2]); acc = acc + p;
        p = q1[1] * bf16hi(kv[2]); acc = acc + p;
        p = q1[2] * bf16lo(kv[3]); acc = acc + p;
        p = q1[3] * bf16hi(kv[3]); acc = acc + p;
      }
      if (half == 1 && lane < 32) {
        const uint32_t t = (wave + 4 * (step >> 1)) * 32 + frow;
        if (t < len) sp[t] = acc * scale;
      }
      wave_sync();
    };
    for (uint32_t step = 0; step < steps; step += 2) {
      process(step, ra);
      process(step + 1, rb);
    }
  }
  // V prefetch: waves 0 and 1 start streaming their first V batch now, so
  // HBM stays busy through the softmax phase.  (The V pass itself is below.)
  unsigned char* vst = stage + (wave & 1) * 8192;  // [64 rows][64 cols] bf16
  const int vrow = lane >> 3, vchunk = lane & 7;
  const uint64_t vcolbase = (uint64_t)(wave & 1) * 64;
  const uint32_t vnb = (len + 63) / 64;
  auto vload = [&](uint32_t bt, u32x4_t* r) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t t = bt * 64 + vrow + 8 * i;
      if (t < len)
        r[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(vb + (uint64_t)t * D + vcolbase + vchunk * 8));
      else
        r[i] = u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  u32x4_t va[8], vbuf[8];
  if (wave < 2 && vnb > 0) vload(0, va);
  __syncthreads();

  // ---------------------------------------------------------------- max
  int lastnan = -1;
  for (uint32_t t = tid; t < len; t += 256)
    if (sp[t] != sp[t]) lastnan = (int)t;
  lastnan = wave_max_i32(lastnan);
  if (lane == 0) red_i[wave] = lastnan;
  __syncthreads();
  int J = red_i[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) J = red_i[w] > J ? red_i[w] : J;

  FirstMax fm{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
  for (uint32_t t = tid; t < len; t += 256)
    if ((int)t > J) fm = first_max_combine(fm, FirstMax{sp[t], t});
  fm = wave_first_max(fm);
  if (lane == 0) {
    red_v[wave] = fm.v;
    red_u[wave] = fm.i;
  }
  __syncthreads();
  FirstMax all{red_v[0], red_u[0]};
#pragma unroll
  for (int w = 1; w < 4; ++w) all = first_max_combine(all, FirstMax{red_v[w], red_u[w]});
  float mx;
  if (len > 0 && J == (int)len - 1)
    mx = sp[len - 1];
  else
    mx = (all.i == 0xFFFFFFFFu) ? __uint_as_float(0xFF800000u) : all.v;
  __syncthreads();  // everyone has read sp[len-1] / red_* before sp is rewritten

  // ---------------------------------------------------------------- exp~, denominator
  for (uint32_t t = tid; t < len; t += 256) {
    const float shifted = sp[t] - mx;
    sp[t] = exp_approx(shifted);
  }
  __syncthreads();
  if (wave == 0) {
    // The one sequential fold: den = (((0 + e_0) + e_1) + ...) in ascending t.
    const float den = serial_sum_wave_long(sp, len);
    if (lane == 0) red_v[0] = den;
  }
  __syncthreads();
  const float den = red_v[0];
  for (uint32_t t = tid; t < len; t += 256) sp[t] = sp[t] / den;
  __syncthreads();

  // ---------------------------------------------------------------- V pass
  if (wave >= 2) return;
  {
    if (vnb > 1) vload(1, vbuf);
    float acc = __uint_as_float(0u);
    const uint16_t* st16 = reinterpret_cast<const uint16_t*>(vst);
    const uint32_t tr_j = (uint32_t)(lane & 15) >> 2;  // row within a group of 4
    const uint32_t tr_col = 16u * ((uint32_t)lane >> 4) + 4u * ((uint32_t)lane & 3);
    auto process = [&](uint32_t bt, u32x4_t* r) {
      set_prio((uint32_t)(qi >> 8) + bt);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        *reinterpret_cast<u32x4_t*>(vst + (vrow + 8 * i) * 128 + vchunk * 16) = r[i];
      wave_sync();
      if (bt + 2 < vnb) vload(bt + 2, r);
      const uint32_t t0 = bt * 64;
      const uint32_t rows = (len - t0) < 64u ? (len - t0) : 64u;
      if (rows == 64) {
        // Four rows of this lane's column per transposing read: lane 4j + a
        // of a 16-lane group addresses row 4u + j, columns 16g + 4a .. +3,
        // and lane i receives column 16g + i of rows 4u .. 4u+3; p comes
        // four at a time (one broadcast read).  Same t-ascending chain.
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const f32x4_t p4 = *reinterpret_cast<const f32x4_t*>(sp + t0 + 4 * u);
          const i16x4_t v4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_i16x4*)(vst + (4 * u + tr_j) * 128 + tr_col * 2));
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float prod = p4[e] * bf16_to_f32((uint16_t)v4[e]);
            acc = acc + prod;
          }
        }
      } else {
        for (uint32_t rr = 0; rr < rows; ++rr) {
          const float prod = sp[t0 + rr] * bf16_to_f32(st16[rr * 64 + lane]);
          acc = acc + prod;
        }
      }
      wave_sync();
    };
    for (uint32_t bt = 0; bt < vnb; bt += 2) {
      process(bt, va);
      if (bt + 1 < vnb) process(bt + 1, vbuf);
    }
    if (OUT_BF16)
      static_cast<uint16_t*>(o)[qi * D + vcolbase + lane] = (uint16_t)f32_to_bf16_bits(acc);
    else
      static_cast<float*>(o)[qi * D + vcolbase + lane] = acc;
  }
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void
catena_attn_decode_bf16_d128(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                             const uint16_t* __restrict__ v, const uint32_t* __restrict__ lens,
                             float* __restrict__ o, uint32_t H, uint32_t L, float scale) {
  attn_body<false>(q, k, v, lens, o, H, L, 1u, scale);
}

// Tq causal queries per sequence (prefill and multi-token steps).
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void
catena_attn_causal_bf16_d128_f32out(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                    const uint16_t* __restrict__ v,
                                    const uint32_t* __restrict__ lens, float* __restrict__ o,
                                    uint32_t H, uint32_t L, uint32_t Tq, float scale) {
  attn_body<false>(q, k, v, lens, o, H, L, Tq, scale);
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void
catena_attn_causal_bf16_d128_bf16out(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                     const uint16_t* __restrict__ v,
                                     const uint32_t* __restrict__ lens, uint16_t* __restrict__ o,
                                     uint32_t H, uint32_t L, uint32_t Tq, float scale) {
  attn_body<true>(q, k, v, lens, o, H, L, Tq, scale);
}
