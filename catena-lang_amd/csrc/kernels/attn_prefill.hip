// Causal KV-cache attention for many queries per sequence (prefill), with
// exactly the per-query arithmetic of attn_decode.hip:
//   s_t = (fold_{d asc} from +0 of q_d * k_{t,d}) * scale
//   m   = f32.max-env fold from -inf;  e_t = exp~(s_t - m)
//   den = fold_{t asc} from +0 of e_t;  p_t = e_t / den
//   o_d = fold_{t asc} from +0 of p_t * v_{t,d}
// (catena-lang/stdlib/matrix.hex:236-256, sum.hex:73-84, nn.hex:59-122,
// math.hex:148-199), so every output is bitwise equal to the decode kernel
// run on that query's prefix.
//
// One workgroup (4 waves) per (batch, head, block of QB = 16 consecutive
// queries); the queries of a block share every K and V row they read.
// Query tq of sequence b attends to the first lens[b] - (Tq - 1 - tq)
// positions (clamped to [0, L]).
//
// Scores: waves take 64-key blocks round robin; lane l owns key kb*64 + l
// and holds its K row in registers (the next block's row is loaded while the
// current one is folded).  The fold over d runs on the matrix cores:
// v_mfma_f32_16x16x1_4b_f32 with A = the 16 queries' q_d (lane l: query
// l % 16, every block) and B = the 64 keys' k_d (lane l: key l) adds
// q_d * k_{t,d} to each of the 16 x 64 accumulators with one rounding, d
// ascending from +0.  The product of two bf16 values is exact in f32 unless
// it leaves the normal range, so one rounding of acc + q_d k_{t,d} is the
// reference's fl(acc + fl(q_d * k_{t,d})) bit for bit whenever every nonzero
// q and k value has magnitude in [2^-63, 2^63) (products in [2^-126, 2^126)).
// That range is checked on the same registers while the MFMAs run (packed
// u16 min / max of the magnitude bits); if any value of the workgroup's q
// rows or K rows lies outside it (tiny, huge, inf or NaN), the workgroup
// recomputes its scores with the VALU fold (v_mul_f32 + v_add_f32 per
// product) before anything reads them.  Scores go to sT[key][query] (row
// stride QB + 1 floats: the per-query reads of softmax are bank-conflict
// free).
// Softmax: per query, the exact parallel form of the max fold (FirstMax,
// common.h) by one wave; exp~ elementwise; the denominators are 16
// independent serial folds, one lane per query; p = e / den elementwise.
// Output: wave w owns queries 4w .. 4w+3 and lane l columns 2l, 2l+1 (8
// accumulators); keys are walked in ascending order through 64-row V blocks
// staged in LDS, the next block's loads in flight while one is folded.  Keys
// below the shortest of the 4 prefixes need no mask; past it, a key beyond a
// query's prefix leaves that accumulator untouched.
#include "common.h"

namespace {
constexpr int D = 128;
constexpr int QS = D + 4;            // qf row stride (floats)
constexpr int QH = D + 8;            // qh row stride (bf16): the MFMA A-operand reads (16 rows,
                                     // 16 bytes each) cover the 64 banks once
constexpr int QB = 16;               // queries per workgroup
constexpr int HALF = QB / 2;         // queries per score item / output thread
constexpr int ST = QB + 1;           // sT row stride (floats)
constexpr int VBLK = 64;             // keys per V stage
constexpr int VSTAGE = VBLK * D * 2; // bytes (bf16)

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Magnitude bits (sign cleared) of two bf16 values; a nonzero value is safe
// for the MFMA fold when its bits lie in [0x2000, 0x5F00): exponent field
// 64 .. 189, i.e. magnitude in [2^-63, 2^63).
constexpr uint32_t kSafeLo = 0x2000u, kSafeHi = 0x5F00u;

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

CATENA_DEV uint32_t query_len(uint32_t lens_b, uint32_t L, uint32_t Tq, uint32_t tq) {
  uint32_t len = lens_b > L ? L : lens_b;
  const uint32_t later = Tq - 1 - tq;
  return len > later ? len - later : 0u;
}
}  // namespace

template <bool OUT_BF16>
CATENA_DEV void prefill_body(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                             const uint16_t* __restrict__ v, const uint32_t* __restrict__ lens,
                             void* __restrict__ o, uint32_t B, uint32_t H, uint32_t L,
                             uint32_t Tq, float scale) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* qf = reinterpret_cast<float*>(smem);                      // [QB][QS]
  uint16_t* qh = reinterpret_cast<uint16_t*>(smem + QB * QS * 4);  // [QB][QH] bf16
  unsigned char* vstage = smem + QB * QS * 4 + QB * QH * 2;        // [VBLK][D] bf16
  float* red = reinterpret_cast<float*>(vstage + VSTAGE);          // [QB] max, [QB] den
  float* sT = red + 3 * QB;                                        // [Lmax][ST] (after qlen)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t BH = B * H;
  const uint32_t nqb = (Tq + QB - 1) / QB;
  // longest query blocks first; the blocks of one (b, h) are BH apart
  const uint32_t qb = nqb - 1 - blockIdx.x / BH;
  const uint32_t bh = blockIdx.x % BH;
  const uint32_t b = bh / H, h = bh % H;
  const uint32_t t0 = qb * QB;
  const uint32_t nq = Tq - t0 < (uint32_t)QB ? Tq - t0 : (uint32_t)QB;
  const uint32_t lb = lens[b];
  // per-query lengths (LDS: indexed with runtime query numbers below); the
  // last query of the block has the longest prefix
  uint32_t* qlen = reinterpret_cast<uint32_t*>(red + 2 * QB);
  if (tid < QB) qlen[tid] = (uint32_t)tid < nq ? query_len(lb, L, Tq, t0 + tid) : 0u;
  const uint32_t lmax = query_len(lb, L, Tq, t0 + nq - 1);

  const uint16_t* kb = k + (uint64_t)bh * L * D;
  const uint16_t* vb = v + (uint64_t)bh * L * D;
  // q rows of this block, widened (rows past nq are zero and never used);
  // `unsafe` notes a value outside the MFMA fold's exact range
  // thread t: row t / 16, values 8 (t % 16) .. +7 (one 16-byte load)
  int unsafe = 0;
  {
    const uint32_t i = (uint32_t)tid / 16, d0 = 8 * ((uint32_t)tid % 16);
    const u32x4_t w = i < nq ? *reinterpret_cast<const u32x4_t*>(q + (((uint64_t)b * Tq + t0 + i) * H + h) * D + d0)
                             : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t lo = w[c] & 0x7FFFu, hi = (w[c] >> 16) & 0x7FFFu;
      unsafe |= (lo != 0u && lo < kSafeLo) || lo >= kSafeHi || (hi != 0u && hi < kSafeLo) || hi >= kSafeHi;
    }
    *reinterpret_cast<f32x4_t*>(qf + i * QS + d0) = f32x4_t{bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1])};
    *reinterpret_cast<f32x4_t*>(qf + i * QS + d0 + 4) = f32x4_t{bf16lo(w[2]), bf16hi(w[2]), bf16lo(w[3]), bf16hi(w[3])};
    *reinterpret_cast<u32x4_t*>(qh + i * QH + d0) = w;
  }
  __syncthreads();

  // ---------------------------------------------------------------- scores
  const uint32_t nkb = (lmax + 63) / 64;
  auto kload = [&](uint32_t kblk, u32x4_t r[D / 8]) {
    const uint32_t j = kblk * 64 + lane;
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(kb + (uint64_t)j * D);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) r[c] = j < lmax ? src[c] : u32x4_t{0u, 0u, 0u, 0u};
  };
  // the MFMA path's form: every lane loads a row in use (a key past lmax
  // reads row lmax - 1; its scores are never stored), so the loads need no
  // branch and the range check sees only rows the scores use
  auto kload_rows = [&](uint32_t kblk, u32x4_t r[D / 8]) {
    const uint32_t j = kblk * 64 + lane;
    const uint32_t jr = j < lmax ? j : lmax - 1u;
    const u32x4_t* src = reinterpret_cast<const u32x4_t*>(kb + (uint64_t)jr * D);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) r[c] = src[c];
  };
  {
    // matrix-core fold: lane l, accumulator r holds key kblk*64 + 16 (r / 4)
    // + l % 16 against query 4 (l / 16) + r % 4
    uint32_t ql[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) ql[u] = qlen[4 * (lane >> 4) + u];
    // lane l's A operand: query l % 16's row, packed bf16 in LDS, eight d
    // values per read, the next read issued before the current MFMAs
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(qh + (lane & 15) * QH);
    u16x2_t mn = {0xFFFF, 0xFFFF}, mx = {0, 0};
    const u16x2_t one = {1, 1};
    u32x4_t raw[D / 8];
    if ((uint32_t)wave < nkb) kload_rows(wave, raw);
    for (uint32_t kblk = wave; kblk < nkb; kblk += 4) {
      u32x4_t cur[D / 8];
#pragma unroll
      for (int c = 0; c < D / 8; ++c) cur[c] = raw[c];
      if (kblk + 4 < nkb) kload_rows(kblk + 4, raw);
      f32x16_t acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = __uint_as_float(0u);
      u32x4_t qnext = qrow[0];
#pragma unroll
      for (int c = 0; c < D / 8; ++c) {
        const u32x4_t qcur = qnext;
        if (c + 1 < D / 8) qnext = qrow[c + 1];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t word = cur[c][w], qword = qcur[w];
          const u16x2_t mag = __builtin_bit_cast(u16x2_t, word & 0x7FFF7FFFu);
          mn = __builtin_elementwise_min(mn, mag - one);
          mx = __builtin_elementwise_max(mx, mag);
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16lo(qword), bf16lo(word), acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16hi(qword), bf16hi(word), acc, 0, 0, 0);
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t j = kblk * 64 + 16 * (r >> 2) + (lane & 15);
        if (j < ql[r & 3]) sT[j * ST + 4 * (lane >> 4) + (r & 3)] = acc[r] * scale;
      }
    }
    // x - 1 wraps a zero to 0xFFFF: a minimum below kSafeLo - 1 is a nonzero
    // value below the range
    const uint32_t lo = mn[0] < mn[1] ? mn[0] : mn[1];
    const uint32_t hi = mx[0] > mx[1] ? mx[0] : mx[1];
    unsafe |= lo < kSafeLo - 1u || hi >= kSafeHi;
  }
  if (__syncthreads_or(unsafe)) {
    // the VALU fold: lane l owns key kb*64 + l, its 128 K values widened into
    // registers once and folded against each of the 16 queries (LDS
    // broadcasts), v_mul_f32 then v_add_f32 per product
    u32x4_t raw[D / 8];
    if ((uint32_t)wave < nkb) kload(wave, raw);
    for (uint32_t kblk = wave; kblk < nkb; kblk += 4) {
      float kf[D];
#pragma unroll
      for (int c = 0; c < D / 8; ++c) {
        kf[8 * c + 0] = bf16lo(raw[c][0]); kf[8 * c + 1] = bf16hi(raw[c][0]);
        kf[8 * c + 2] = bf16lo(raw[c][1]); kf[8 * c + 3] = bf16hi(raw[c][1]);
        kf[8 * c + 4] = bf16lo(raw[c][2]); kf[8 * c + 5] = bf16hi(raw[c][2]);
        kf[8 * c + 6] = bf16lo(raw[c][3]); kf[8 * c + 7] = bf16hi(raw[c][3]);
      }
      if (kblk + 4 < nkb) kload(kblk + 4, raw);
      const uint32_t j = kblk * 64 + lane;
#pragma unroll 1
      for (int i = 0; i < QB; ++i) {
        const uint32_t li = qlen[i];
        if (kblk * 64 >= li) continue;
        const f32x4_t* q4 = reinterpret_cast<const f32x4_t*>(qf + i * QS);
        float acc = __uint_as_float(0u);
#pragma unroll
        for (int c = 0; c < D / 4; ++c) {
          const f32x4_t qq = q4[c];
          float p;
          p = qq[0] * kf[4 * c + 0]; acc = acc + p;
          p = qq[1] * kf[4 * c + 1]; acc = acc + p;
          p = qq[2] * kf[4 * c + 2]; acc = acc + p;
          p = qq[3] * kf[4 * c + 3]; acc = acc + p;
        }
        if (j < li) sT[j * ST + i] = acc * scale;
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- max per query
  // Wave w takes queries w, w + 4, w + 8, w + 12 in one pass over the
  // scores: per lane and query, the last NaN position and the first max of
  // every value the lane read (positions ascending).  Without a NaN in the
  // query's prefix, the first-max combine of those over the lanes
  // (associative and commutative) is the sequential fold's result, as in the
  // two-pass form; a query with a NaN takes that form (first max after the
  // last NaN, or the NaN itself when it is the last position).
  {
    uint32_t len4[4], lmx = 0;
    int ln4[4];
    FirstMax fm4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      len4[u] = qlen[wave + 4 * u];
      lmx = len4[u] > lmx ? len4[u] : lmx;
      ln4[u] = -1;
      fm4[u] = FirstMax{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
    }
    // per lane the positions ascend, so its first maximum is kept by a
    // strict comparison (a NaN never replaces it; a query with one takes the
    // two-pass form below; a lane holding only -inf stays empty, which the
    // combine treats as -inf)
    float bv[4];
    uint32_t bi[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      bv[u] = __uint_as_float(0xFF800000u);
      bi[u] = 0xFFFFFFFFu;
    }
    for (uint32_t t = lane; t < lmx; t += 64) {
      const float* row = sT + t * ST + wave;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (t < len4[u]) {
          const float sv = row[4 * u];
          if (sv != sv) ln4[u] = (int)t;
          if (sv > bv[u]) {
            bv[u] = sv;
            bi[u] = t;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) fm4[u] = FirstMax{bv[u], bi[u]};
    // the four queries' butterflies interleaved (independent shuffle chains)
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int o = __shfl_xor(ln4[u], off, 64);
        ln4[u] = o > ln4[u] ? o : ln4[u];
        FirstMax b;
        b.v = __shfl_xor(fm4[u].v, off, 64);
        b.i = (uint32_t)__shfl_xor((int)fm4[u].i, off, 64);
        fm4[u] = first_max_combine(fm4[u], b);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = wave + 4 * u;
      const uint32_t len = len4[u];
      const int J = ln4[u];
      FirstMax fm;
      if (J < 0) {
        fm = fm4[u];
      } else {
        fm = FirstMax{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
        for (uint32_t t = lane; t < len; t += 64)
          if ((int)t > J) fm = first_max_combine(fm, FirstMax{sT[t * ST + i], t});
        fm = wave_first_max(fm);
      }
      if (lane == 0) {
        float mx;
        if (len > 0 && J == (int)len - 1)
          mx = sT[(len - 1) * ST + i];
        else
          mx = fm.i == 0xFFFFFFFFu ? __uint_as_float(0xFF800000u) : fm.v;
        red[i] = mx;
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- exp~
  // four elements per thread in flight (each element's arithmetic unchanged)
  for (uint32_t e0 = tid; e0 < lmax * QB; e0 += 4 * 256) {
    float sv[4], mv[4];
    bool live[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t e = e0 + 256u * u, t = e / QB, i = e % QB;
      live[u] = e < lmax * QB && t < qlen[i];
      sv[u] = live[u] ? sT[t * ST + i] : 0.0f;
      mv[u] = red[i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t e = e0 + 256u * u, t = e / QB, i = e % QB;
      if (live[u]) {
        const float shifted = sv[u] - mv[u];
        sT[t * ST + i] = exp_approx(shifted);
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- denominators
  if (tid < QB) {
    // lane i: den_i = (((0 + e_0) + e_1) + ...), t ascending; the next 32
    // (short prefixes: 8) values are read before the current ones are added
    const int i = tid;
    const uint32_t len = qlen[i];
    float den = __uint_as_float(0u);
    uint32_t t = 0;
    if (len >= 64) {
      float cur[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) cur[u] = sT[u * ST + i];
      for (t = 32; t + 32 <= len; t += 32) {
        float nxt[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) nxt[u] = sT[(t + u) * ST + i];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 32; ++u) den = den + cur[u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 32; ++u) cur[u] = nxt[u];
      }
#pragma unroll
      for (int u = 0; u < 32; ++u) den = den + cur[u];
    } else if (len >= 16) {
      float cur[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = sT[u * ST + i];
      for (t = 8; t + 8 <= len; t += 8) {
        float nxt[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) nxt[u] = sT[(t + u) * ST + i];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 8; ++u) den = den + cur[u];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) den = den + cur[u];
    }
    for (; t < len; ++t) den = den + sT[t * ST + i];
    red[QB + i] = den;
  }
  __syncthreads();
  for (uint32_t e0 = tid; e0 < lmax * QB; e0 += 4 * 256) {
    float sv[4], dv[4];
    bool live[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t e = e0 + 256u * u, t = e / QB, i = e % QB;
      live[u] = e < lmax * QB && t < qlen[i];
      sv[u] = live[u] ? sT[t * ST + i] : 0.0f;
      dv[u] = red[QB + i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t e = e0 + 256u * u, t = e / QB, i = e % QB;
      if (live[u]) sT[t * ST + i] = sv[u] / dv[u];
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- P V
  const int qg = wave;                       // queries 4qg .. 4qg+3
  const uint32_t cp = (uint32_t)lane;        // columns 2cp, 2cp+1
  uint32_t glen[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) glen[u] = qlen[4 * qg + u];
  // Prefixes grow with the query, but queries past nq (a last block's
  // padding) have length 0: the longest of the four is their maximum, not
  // the last one's (with two or three real queries in the wave, the last
  // slot is padding).  The shortest is the first's (padding only follows).
  uint32_t lmax4 = glen[0];
#pragma unroll
  for (int u = 1; u < 4; ++u) lmax4 = glen[u] > lmax4 ? glen[u] : lmax4;
  const uint32_t lmin4 = glen[0];
  float acc0[4], acc1[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) acc0[u] = acc1[u] = __uint_as_float(0u);

  const uint32_t nvb = (lmax + VBLK - 1) / VBLK;
  // cooperative V stage: 64 rows x 256 B = 1024 x 16 B, 4 per thread
  auto vload = [&](uint32_t blk, u32x4_t r[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t c = tid + 256 * u;  // 16-byte chunk
      const uint32_t row = c >> 4, part = c & 15;
      const uint32_t t = blk * VBLK + row;
      r[u] = t < lmax ? *reinterpret_cast<const u32x4_t*>(vb + (uint64_t)t * D + part * 8)
                      : u32x4_t{0u, 0u, 0u, 0u};
    }
  };
  u32x4_t vr[4];
  if (nvb > 0) vload(0, vr);
  const uint32_t* vs32 = reinterpret_cast<const uint32_t*>(vstage);
  for (uint32_t blk = 0; blk < nvb; ++blk) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      reinterpret_cast<u32x4_t*>(vstage)[tid + 256 * u] = vr[u];
    __syncthreads();
    if (blk + 1 < nvb) vload(blk + 1, vr);
    const uint32_t tb = blk * VBLK;
    const uint32_t rows = lmax - tb < (uint32_t)VBLK ? lmax - tb : (uint32_t)VBLK;
    const uint32_t full = lmin4 > tb ? (lmin4 - tb < rows ? lmin4 - tb : rows) : 0u;
    const uint32_t part = lmax4 > tb ? (lmax4 - tb < rows ? lmax4 - tb : rows) : 0u;
    for (uint32_t r = 0; r < full; ++r) {
      const uint32_t w = vs32[r * (D / 2) + cp];
      const float v0 = bf16lo(w), v1 = bf16hi(w);
      const float* prow = sT + (tb + r) * ST + 4 * qg;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float pu = prow[u];
        const float x0 = pu * v0, x1 = pu * v1;
        acc0[u] = acc0[u] + x0;
        acc1[u] = acc1[u] + x1;
      }
    }
    for (uint32_t r = full; r < part; ++r) {
      const uint32_t t = tb + r;
      const uint32_t w = vs32[r * (D / 2) + cp];
      const float v0 = bf16lo(w), v1 = bf16hi(w);
      const float* prow = sT + t * ST + 4 * qg;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (t < glen[u]) {
          const float pu = prow[u];
          const float x0 = pu * v0, x1 = pu * v1;
          acc0[u] = acc0[u] + x0;
          acc1[u] = acc1[u] + x1;
        }
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t qi = 4 * qg + u;
    if (qi >= nq) continue;
    const uint64_t off = (((uint64_t)b * Tq + t0 + qi) * H + h) * D + 2 * cp;
    if (OUT_BF16)
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(o) + off) = pack_bf16x2(acc0[u], acc1[u]);
    else
      *reinterpret_cast<float2*>(static_cast<float*>(o) + off) = make_float2(acc0[u], acc1[u]);
  }
}

// grid = B * H * ceil(Tq / 16), block = 256, dynamic LDS =
// 16*132*4 + 16*136*2 + 64*128*2 + 3*16*4 + Lmax*17*4 with Lmax >= min(max lens, L).
extern "C" __global__ __launch_bounds__(256) void catena_attn_prefill_bf16_d128_f32out(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint32_t* __restrict__ lens, float* __restrict__ o, uint32_t B, uint32_t H, uint32_t L,
    uint32_t Tq, float scale) {
  prefill_body<false>(q, k, v, lens, o, B, H, L, Tq, scale);
}

extern "C" __global__ __launch_bounds__(256) void catena_attn_prefill_bf16_d128_bf16out(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint32_t* __restrict__ lens, uint16_t* __restrict__ o, uint32_t B, uint32_t H, uint32_t L,
    uint32_t Tq, float scale) {
  prefill_body<true>(q, k, v, lens, o, B, H, L, Tq, scale);
}
