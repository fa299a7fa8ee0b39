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
// and holds its K row in registers (chunk c of the next block's row is
// loaded as soon as chunk c of the current one is folded).  The fold over d
// runs on the matrix cores: v_mfma_f32_16x16x1_4b_f32 with A = the 16
// queries' q_d (lane l: query l % 16, every block) and B = the 64 keys'
// k_d (lane l: key l) adds q_d * k_{t,d} to each of the 16 x 64
// accumulators with one rounding, d ascending from +0.  The product of two
// bf16 values is exact in f32 unless it leaves the normal range, so one
// rounding of acc + q_d k_{t,d} is the reference's fl(acc + fl(q_d *
// k_{t,d})) bit for bit whenever every nonzero q and k value has magnitude
// in [2^-63, 2^63) (products in [2^-126, 2^126)).  That range is checked on
// the same registers while the MFMAs run (packed u16 min / max of the
// magnitude bits); if any value of the workgroup's q rows or K rows lies
// outside it (tiny, huge, inf or NaN), the workgroup recomputes its scores
// with the VALU fold (v_mul_f32 + v_add_f32 per product) before anything
// reads them.  Scores go to sT[key][query] (row stride QB + 1 floats: the
// per-query reads of softmax are bank-conflict free; rows for whole 64-key
// blocks).
// Softmax: per query, the exact parallel form of the max fold (FirstMax,
// common.h): each lane tracks the first maximum and the last NaN of the
// scores it produces, rows of 16 lanes combine them by DPP and the max
// phase combines the four waves' partials; exp~ elementwise; the
// denominators are 16 independent serial folds, one lane per query;
// p = e / den elementwise.
// Output: wave w owns columns 32w .. 32w + 31 of all 16 queries.  The
// products p_t * v_{t,c} come from v_mfma_f32_16x16x1_4b_f32 with a zero
// accumulator (one product, one rounding: fl(p * v)), four keys per
// instruction; the VALU adds them to the running sums in ascending key
// order.  LDS holds the q rows (bf16), the per-query scalars, the max
// partials and the score matrix only (V is read by each wave itself), so
// three workgroups share a CU at the C5 shape.  Keys below the shortest
// prefix of the block need no mask; past it, a key beyond a query's prefix
// leaves that query's sums untouched.
#include "common.h"

namespace {
constexpr int D = 128;
constexpr int QH = D + 8;            // qh row stride (bf16): the MFMA A-operand reads (16 rows,
                                     // 16 bytes each) cover the 64 banks once
constexpr int QB = 16;               // queries per workgroup
constexpr int HALF = QB / 2;         // queries per score item / output thread
constexpr int ST = QB + 1;           // sT row stride (floats)

typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

// Magnitude bits (sign cleared) of two bf16 values; a nonzero value is safe
// for the MFMA fold when its bits lie in [0x2000, 0x5F00): exponent field
// 64 .. 189, i.e. magnitude in [2^-63, 2^63).
constexpr uint32_t kSafeLo = 0x2000u, kSafeHi = 0x5F00u;

// Raw buffer descriptor word 3 (stride 0, bounds-checked by byte offset)
constexpr int kRsrcWord3 = 0x00020000;

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

// a combined with the value CTRL's DPP row pattern brings to this lane
template <int CTRL>
CATENA_DEV FirstMax row_first_max(FirstMax a) {
  FirstMax b;
  b.v = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a.v), CTRL, 0xF, 0xF, false));
  b.i = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)a.i, CTRL, 0xF, 0xF, false);
  return first_max_combine(a, b);
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
  uint16_t* qh = reinterpret_cast<uint16_t*>(smem);                // [QB][QH] bf16
  float* red = reinterpret_cast<float*>(smem + QB * QH * 2);       // [QB] max, [QB] den
  float* part = red + 3 * QB;  // [3][4 waves][QB]: first-max value, its index, last NaN
  float* sT = part + 3 * 4 * QB;                                   // [Lmax][ST]

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
  // q rows of this block, bf16 (rows past nq are zero and never used);
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
  // the MFMA path's form: buffer loads over the block's rows (a key past
  // lmax reads zeros, which the range check passes and whose scores are
  // never used), so the loads need no branch
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)kb, (short)0,
                                        __builtin_amdgcn_readfirstlane((int)(lmax * (uint32_t)D * 2u)), kRsrcWord3);
  auto kchunk = [&](uint32_t j, int c) -> u32x4_t {
    return __builtin_amdgcn_raw_buffer_load_b128(krs, (int)(j * (uint32_t)D * 2u) + 16 * c, 0, 0);
  };
  {
    // matrix-core fold: lane l, accumulator r holds key kblk*64 + 16 (r / 4)
    // + l % 16 against query 4 (l / 16) + r % 4.  Each lane also keeps, per
    // query, the first maximum and the last NaN position of the scores it
    // produces (positions ascend per lane), the max phase's partials
    // lane l's A operand: query l % 16's row, packed bf16 in LDS, eight d
    // values per read, the next read issued before the current MFMAs
    const u32x4_t* qrow = reinterpret_cast<const u32x4_t*>(qh + (lane & 15) * QH);
    u16x2_t mn = {0xFFFF, 0xFFFF}, mx = {0, 0};
    const u16x2_t one = {1, 1};
    uint32_t ql[4];
    float bv[4];
    uint32_t bi[4];
    int ln[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ql[u] = qlen[4 * (lane >> 4) + u];
      bv[u] = __uint_as_float(0xFF800000u);
      bi[u] = 0xFFFFFFFFu;
      ln[u] = -1;
    }
    // the K row chunks rotate through one set of registers: chunk c of the
    // wave's next block (zeros past the rows) is loaded as soon as chunk c
    // of the current one has been folded, a whole block ahead of its use
    u32x4_t raw[D / 8];
#pragma unroll
    for (int c = 0; c < D / 8; ++c) raw[c] = kchunk((uint32_t)wave * 64 + lane, c);
    for (uint32_t kblk = wave; kblk < nkb; kblk += 4) {
      const uint32_t jn = (kblk + 4) * 64 + lane;
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
          const uint32_t word = raw[c][w], qword = qcur[w];
          const u16x2_t mag = __builtin_bit_cast(u16x2_t, word & 0x7FFF7FFFu);
          mn = __builtin_elementwise_min(mn, mag - one);
          mx = __builtin_elementwise_max(mx, mag);
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16lo(qword), bf16lo(word), acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x1f32(bf16hi(qword), bf16hi(word), acc, 0, 0, 0);
        }
        raw[c] = kchunk(jn, c);
        // one chunk at a time: its conversions and range check are not
        // hoisted ahead, nor the next block's load of it sunk behind
        __builtin_amdgcn_sched_barrier(0);
      }
      // scores of the block (sT has rows for every key of the last block;
      // one past a query's prefix is never read), and the running first
      // maximum (strict comparison: the first one, never a NaN) and last NaN
      // of the positions inside each query's prefix
      float* base = sT + (kblk * 64 + (lane & 15)) * ST + 4 * (lane >> 4);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const uint32_t j = kblk * 64 + 16 * (r >> 2) + (lane & 15);
        const float sv = acc[r] * scale;
        base[16 * (r >> 2) * ST + (r & 3)] = sv;
        const int u = r & 3;
        const bool in = j < ql[u];
        ln[u] = in && sv != sv ? (int)j : ln[u];
        const bool up = in && sv > bv[u];
        bv[u] = up ? sv : bv[u];
        bi[u] = up ? j : bi[u];
      }
    }
    // the 16 lanes of a row hold the same 4 queries: combine them (rotations
    // by 8, 4, 2, 1 within the row give every lane all 16), then one lane per
    // row writes the wave's partials
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      FirstMax f{bv[u], bi[u]};
      f = row_first_max<0x128>(f);
      f = row_first_max<0x124>(f);
      f = row_first_max<0x122>(f);
      f = row_first_max<0x121>(f);
      int n = ln[u];
      n = max(n, __builtin_amdgcn_update_dpp(0, n, 0x128, 0xF, 0xF, false));
      n = max(n, __builtin_amdgcn_update_dpp(0, n, 0x124, 0xF, 0xF, false));
      n = max(n, __builtin_amdgcn_update_dpp(0, n, 0x122, 0xF, 0xF, false));
      n = max(n, __builtin_amdgcn_update_dpp(0, n, 0x121, 0xF, 0xF, false));
      if ((lane & 15) == 0) {
        const int qi = 4 * (lane >> 4) + u;
        part[wave * QB + qi] = f.v;
        part[4 * QB + wave * QB + qi] = __uint_as_float(f.i);
        part[8 * QB + wave * QB + qi] = __int_as_float(n);
      }
    }
    // x - 1 wraps a zero to 0xFFFF: a minimum below kSafeLo - 1 is a nonzero
    // value below the range
    const uint32_t lo = mn[0] < mn[1] ? mn[0] : mn[1];
    const uint32_t hi = mx[0] > mx[1] ? mx[0] : mx[1];
    unsafe |= lo < kSafeLo - 1u || hi >= kSafeHi;
  }
  const bool refold = __syncthreads_or(unsafe) != 0;
  if (refold) {
    // the VALU fold: lane l owns key kb*64 + l, its 128 K values in registers
    // (bf16 pairs, widened at each use) folded against each of the 16
    // queries (LDS broadcasts of the bf16 q rows), v_mul_f32 then v_add_f32
    // per product, d ascending
    for (uint32_t kblk = wave; kblk < nkb; kblk += 4) {
      u32x4_t raw[D / 8];
      kload(kblk, raw);
      const uint32_t j = kblk * 64 + lane;
#pragma unroll 1
      for (int i = 0; i < QB; ++i) {
        const uint32_t li = qlen[i];
        if (kblk * 64 >= li) continue;
        // keeps the widened K values out of registers across queries (the
        // compiler would otherwise hoist all 128 of them out of this loop)
#pragma unroll
        for (int c = 0; c < D / 8; ++c) asm volatile("" : "+v"(raw[c]));
        const u32x4_t* q8 = reinterpret_cast<const u32x4_t*>(qh + i * QH);
        float acc = __uint_as_float(0u);
#pragma unroll
        for (int c = 0; c < D / 8; ++c) {
          const u32x4_t qq = q8[c];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            float p;
            p = bf16lo(qq[w]) * bf16lo(raw[c][w]); acc = acc + p;
            p = bf16hi(qq[w]) * bf16hi(raw[c][w]); acc = acc + p;
          }
          // eight products in flight at a time, not all 128
          __builtin_amdgcn_sched_barrier(0);
        }
        if (j < li) sT[j * ST + i] = acc * scale;
      }
    }
  }
  __syncthreads();

  // ---------------------------------------------------------------- max per query
  // Wave w takes queries w, w + 4, w + 8, w + 12: the last NaN position and
  // the first max of the query's scores, from the four waves' partials of
  // the matrix-core fold, or (after a VALU refold) from one pass over the
  // scores in which each lane keeps them for the positions it reads
  // (ascending).  Without a NaN in the query's prefix, the first-max combine
  // of those (associative and commutative) is the sequential fold's result,
  // as in the two-pass form; a query with a NaN takes that form (first max
  // after the last NaN, or the NaN itself when it is the last position).
  {
    uint32_t len4[4];
    int ln4[4];
    FirstMax fm4[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) len4[u] = qlen[wave + 4 * u];
    if (!refold) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int i = wave + 4 * u;
        FirstMax f{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
        int n = -1;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          f = first_max_combine(f, FirstMax{part[w * QB + i], __float_as_uint(part[4 * QB + w * QB + i])});
          const int nw = __float_as_int(part[8 * QB + w * QB + i]);
          n = nw > n ? nw : n;
        }
        fm4[u] = f;
        ln4[u] = n;
      }
    } else {
      uint32_t lmx = 0;
#pragma unroll
      for (int u = 0; u < 4; ++u) lmx = len4[u] > lmx ? len4[u] : lmx;
      // per lane the positions ascend, so its first maximum is kept by a
      // strict comparison (a NaN never replaces it; a lane holding only
      // -inf stays empty, which the combine treats as -inf)
      float bv[4];
      uint32_t bi[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        bv[u] = __uint_as_float(0xFF800000u);
        bi[u] = 0xFFFFFFFFu;
        ln4[u] = -1;
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
  // Wave w owns output columns 32w .. 32w + 31 of the 16 queries.  For each
  // group of 4 keys t .. t + 3, two v_mfma_f32_16x16x1_4b_f32 with a zero
  // accumulator form the 16 x 16 x 4 products (K = 1: one product, one
  // rounding, so each is fl(p * v), the reference's product; a -0 product
  // comes out +0, which no add below can tell apart: every sum starts at +0
  // and never becomes -0): block b = key t + b, row i = query i (A: lane
  // 16b + i holds p[i][t + b]), column j = column pair j of the wave (B:
  // lane 16b + j holds v[t + b][32w + 2j], the second MFMA the odd column).
  // Lane l receives in register 4kk + u the product of key t + kk, query
  // 4(l / 16) + u and its column pair l % 16, and adds it to that query's
  // two sums on the VALU, keys in ascending order (a key past the query's
  // prefix is skipped).
  const uint32_t jp = (uint32_t)lane & 15, kq = (uint32_t)lane >> 4;
  uint32_t glen[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) glen[u] = qlen[4 * kq + u];
  // every real query of the block sees at least qlen[0] keys (padding rows'
  // sums are never stored)
  const uint32_t ng = (lmax + 3) / 4, nfull = qlen[0] / 4;
  float s0[4], s1[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) s0[u] = s1[u] = __uint_as_float(0u);
  // V words by range-checked buffer loads (keys past lmax read zeros),
  // eight groups ahead of their use
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)vb, (short)0,
                                        __builtin_amdgcn_readfirstlane((int)(lmax * (uint32_t)D * 2u)), kRsrcWord3);
  const int voff = (int)((kq * D + 32 * (uint32_t)wave + 2 * jp) * 2u);
  auto vload = [&](uint32_t t) -> uint32_t {
    return __builtin_amdgcn_raw_buffer_load_b32(vrs, voff + (int)(t * (uint32_t)D * 2u), 0, 0);
  };
  const float* pcol = sT + kq * ST + jp;  // p[jp][t + kq] at pcol[t * ST]
  const f32x16_t zero16 = {};
  uint32_t vw[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) vw[i] = vload(4u * i);
  for (uint32_t g = 0; g < ng; g += 8) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t t = 4 * (g + i);
      const uint32_t w = vw[i];
      vw[i] = vload(t + 32);
      if (g + i < ng) {
        const float pv = pcol[t * ST];
        const f32x16_t x0 = __builtin_amdgcn_mfma_f32_16x16x1f32(pv, bf16lo(w), zero16, 0, 0, 0);
        const f32x16_t x1 = __builtin_amdgcn_mfma_f32_16x16x1f32(pv, bf16hi(w), zero16, 0, 0, 0);
        if (g + i < nfull) {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              s0[u] = s0[u] + x0[4 * kk + u];
              s1[u] = s1[u] + x1[4 * kk + u];
            }
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const bool in = t + kk < glen[u];
              s0[u] = in ? s0[u] + x0[4 * kk + u] : s0[u];
              s1[u] = in ? s1[u] + x1[4 * kk + u] : s1[u];
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint32_t qi = 4 * kq + u;
    if (qi >= nq) continue;
    const uint64_t off = (((uint64_t)b * Tq + t0 + qi) * H + h) * D + 32 * (uint32_t)wave + 2 * jp;
    if (OUT_BF16)
      *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(o) + off) = pack_bf16x2(s0[u], s1[u]);
    else
      *reinterpret_cast<float2*>(static_cast<float*>(o) + off) = make_float2(s0[u], s1[u]);
  }
}

// Four waves per SIMD: the register budget is then 128 (the matrix-core
// results in ordinary VGPRs, no AGPR copies before the VALU adds; one value
// spilled to 8 bytes of scratch), so four workgroups share a CU when the
// score buffer allows (up to 512 rows): C5 prefill 256 -> 234 us.
// grid = B * H * ceil(Tq / 16), block = 256, dynamic LDS =
// 16*136*2 + 3*16*4 + 3*4*16*4 + R*17*4 with R >= min(max lens, L) rounded up
// to a multiple of 64 (the score rows of whole 64-key blocks).
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void catena_attn_prefill_bf16_d128_f32out(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint32_t* __restrict__ lens, float* __restrict__ o, uint32_t B, uint32_t H, uint32_t L,
    uint32_t Tq, float scale) {
  prefill_body<false>(q, k, v, lens, o, B, H, L, Tq, scale);
}

extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void catena_attn_prefill_bf16_d128_bf16out(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
    const uint32_t* __restrict__ lens, uint16_t* __restrict__ o, uint32_t B, uint32_t H, uint32_t L,
    uint32_t Tq, float scale) {
  prefill_body<true>(q, k, v, lens, o, B, H, L, Tq, scale);
}
