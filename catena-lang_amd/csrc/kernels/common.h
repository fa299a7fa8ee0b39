// Device-side helpers shared by the gfx950 kernels.
//
// Every kernel in this directory is compiled with -ffp-contract=off
// -fno-fast-math (build.py), the flag contract of the reference's generated
// module (catena-lang/src/runtime/artifact.rs:59-71): `a * b + c` stays a
// separately rounded multiply and add, never an FMA.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define CATENA_DEV __device__ __forceinline__

// catena_u32_bitcast_f32 / catena_f32_bitcast_u32
// (catena-lang/src/codegen/prelude.rs:64-80)
CATENA_DEV float u32_as_f32(uint32_t b) { return __uint_as_float(b); }
CATENA_DEV uint32_t f32_as_u32(float f) { return __float_as_uint(f); }

// Exact bf16 -> f32 widening of the low / high half of a packed dword.
CATENA_DEV float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
CATENA_DEV float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
CATENA_DEV float bf16_to_f32(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

// f32 -> bf16 round-to-nearest-even; NaN keeps sign and top payload and is
// made quiet.  Integer formulation so the CPU oracle (or_f32_to_bf16) and the
// device agree bit for bit.
CATENA_DEV uint32_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x0040u;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return u >> 16;
}

CATENA_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// f32.round-to-u32 = (uint32_t)nearbyintf(x) (catena-lang/src/codegen/
// gpu.rs:642-655), with the device conversion's defined behaviour spelled
// out: NaN and values <= 0 give 0, values >= 2^32 saturate.
CATENA_DEV uint32_t round_to_u32(float x) {
  const float r = __builtin_rintf(x);
  // branch-free: max(NaN, 0) = 0 and max(negative, 0) = 0; below 2^32 the
  // conversion is exact; at or above 2^32 the result saturates.
  const float c = __builtin_fminf(__builtin_fmaxf(r, 0.0f), 4294967040.0f);
  const uint32_t k = (uint32_t)c;
  return (r >= 4294967296.0f) ? 0xFFFFFFFFu : k;
}

// math.exp-approx-nonneg (catena-lang/stdlib/math.hex:148-183); one IEEE
// operation per hexpr node, operands in source order.
CATENA_DEV float exp_approx_nonneg(float x) {
  const float inv_ln2 = u32_as_f32(0x3FB8AA3Bu);
  const float ln2_hi = u32_as_f32(0x3F317200u);
  const float ln2_lo = u32_as_f32(0x35BFBE8Eu);
  const float c0 = u32_as_f32(0x3F7FF8FCu);
  const float c1 = u32_as_f32(0x3F809C7Eu);
  const float c2 = u32_as_f32(0x3EEF1187u);
  const float c3 = u32_as_f32(0x3E738A8Bu);
  float scaled = x * inv_ln2;
  uint32_t k_u32 = round_to_u32(scaled);
  float k_f32 = (float)k_u32;
  float k_ln2_hi = k_f32 * ln2_hi;
  float k_ln2_lo = k_f32 * ln2_lo;
  float r1 = x - k_ln2_hi;
  float xr = r1 - k_ln2_lo;
  float xr_c3 = xr * c3;
  float p2 = c2 + xr_c3;
  float xr_p2 = xr * p2;
  float p1 = c1 + xr_p2;
  float xr_p1 = xr * p1;
  float poly = c0 + xr_p1;
  uint32_t biased = k_u32 + 0x7Fu;           // u32.add wraps
  uint32_t pow2_bits = biased * 0x00800000u;  // u32.mul wraps
  return poly * u32_as_f32(pow2_bits);
}

// math.exp-approx (catena-lang/stdlib/math.hex:185-199)
CATENA_DEV float exp_approx(float x) {
  const float zero = (float)0u;
  const float one = u32_as_f32(0x3F800000u);
  float neg_x = -x;
  bool is_negative = x < zero;
  float magnitude = is_negative ? neg_x : x;
  float base = exp_approx_nonneg(magnitude);
  float reciprocal = one / base;  // correctly rounded (no fast-math)
  return is_negative ? reciprocal : base;
}

// math.sqrt (catena-lang/stdlib/math.hex:235-272): six Newton steps from
// guess0 = (x < 1) ? 1 : x; non-positive inputs give +0.
CATENA_DEV float sqrt_newton(float x) {
  const float zero = (float)0u;
  const float one = u32_as_f32(0x3F800000u);
  const float half = u32_as_f32(0x3F000000u);
  const bool lt_one = x < one;
  float g = lt_one ? one : x;
#pragma unroll
  for (int it = 0; it < 6; ++it) {
    const float ratio = x / g;
    const float sum = g + ratio;
    g = sum * half;
  }
  const bool is_nonpositive = x <= zero;
  return is_nonpositive ? zero : g;
}

// nn.sigmoid / nn.silu (catena-lang/stdlib/nn.hex:1-21)
CATENA_DEV float sigmoid_approx(float x) {
  const float one = 1.0f;
  const float neg_x = -x;
  const float e = exp_approx(neg_x);
  const float den = one + e;
  return one / den;
}
CATENA_DEV float silu_approx(float x) {
  const float gate = sigmoid_approx(x);
  return x * gate;
}

// math.sin-approx / math.cos-approx (catena-lang/stdlib/math.hex:1-47)
CATENA_DEV float sin_taylor(float x) {
  const float x2 = x * x, x3 = x2 * x, x5 = x3 * x2, x7 = x5 * x2;
  const float a = x3 / (float)6u, b = x5 / (float)120u, c = x7 / (float)5040u;
  const float p1 = x - a;
  const float p2 = p1 + b;
  return p2 - c;
}
CATENA_DEV float cos_taylor(float x) {
  const float x2 = x * x, x4 = x2 * x2, x6 = x4 * x2;
  const float a = x2 / (float)2u, b = x4 / (float)24u, c = x6 / (float)720u;
  const float p1 = (float)1u - a;
  const float p2 = p1 + b;
  return p2 - c;
}
// Cody-Waite quadrant evaluation of math.sin-approx-full-nonneg
// (catena-lang/stdlib/math.hex:52-88); shift = 1 gives the cosine this
// build defines (the quadrant advanced by one: cos x = sin(x + pi/2)).
CATENA_DEV float quadrant_eval(float x, uint32_t shift) {
  const float inv_pio2 = u32_as_f32(0x3F22F983u);
  const float pio2_hi = u32_as_f32(0x3FC90FDAu);
  const float pio2_lo = u32_as_f32(0x33A22168u);
  const float scaled = x * inv_pio2;
  const uint32_t n_u32 = round_to_u32(scaled);
  const float n_f = (float)n_u32;
  const float n_hi = n_f * pio2_hi;
  const float n_lo = n_f * pio2_lo;
  const float r1 = x - n_hi;
  const float r = r1 - n_lo;
  const float sin_r = sin_taylor(r);
  const float cos_r = cos_taylor(r);
  const float neg_sin = -sin_r, neg_cos = -cos_r;
  const uint32_t quadrant = (n_u32 + shift) & 3u;
  const float q23 = quadrant == 2u ? neg_sin : neg_cos;
  const float q123 = quadrant == 1u ? cos_r : q23;
  return quadrant == 0u ? sin_r : q123;
}
// math.sin-approx-full (catena-lang/stdlib/math.hex:90-103)
CATENA_DEV float sin_full(float x) {
  const bool is_negative = x < (float)0u;
  const float magnitude = is_negative ? -x : x;
  const float base = quadrant_eval(magnitude, 0u);
  return is_negative ? -base : base;
}
CATENA_DEV float cos_full(float x) {
  const bool is_negative = x < (float)0u;
  const float magnitude = is_negative ? -x : x;
  return quadrant_eval(magnitude, 1u);
}

// The sequential left fold ((0 + s[0]) + s[1]) + ... over n floats in LDS
// (16-byte aligned), by one lane.  The next 32 values are requested before
// the current 32 are added (the scheduling barrier keeps the compiler from
// sinking those reads below the adds), so LDS latency stays off the
// dependency chain.
CATENA_DEV float serial_sum_lds(const float* s, uint32_t n) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  float acc = __uint_as_float(0u);
  const uint32_t n4 = n / 4;
  const f4* s4 = reinterpret_cast<const f4*>(s);
  uint32_t i = 0;
  if (n4 >= 8) {
    f4 cur[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = s4[u];
    for (i = 8; i + 8 <= n4; i += 8) {
      f4 nxt[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) nxt[u] = s4[i + u];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        acc = acc + cur[u][0];
        acc = acc + cur[u][1];
        acc = acc + cur[u][2];
        acc = acc + cur[u][3];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < 8; ++u) cur[u] = nxt[u];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc = acc + cur[u][0];
      acc = acc + cur[u][1];
      acc = acc + cur[u][2];
      acc = acc + cur[u][3];
    }
  }
  for (; i < n4; ++i) {
    const f4 e = s4[i];
    acc = acc + e[0];
    acc = acc + e[1];
    acc = acc + e[2];
    acc = acc + e[3];
  }
  for (uint32_t t = n4 * 4; t < n; ++t) acc = acc + s[t];
  return acc;
}

// The same sequential fold computed by one whole wave (all 64 lanes call
// it; every lane gets the result).  Each 2048-value chunk is spread over
// the lanes, lane L holding values 32L .. 32L+31 in registers; the running
// sum then passes from lane to lane through a scalar register while the lane
// owning the next 32 values adds them in order with the others masked off.
// The dependency chain is one v_add_f32 per value with no memory access on
// it (a single lane reading LDS per value is several times slower).
CATENA_DEV float serial_sum_wave(const float* s, uint32_t n) {
  const uint32_t lane = threadIdx.x & 63u;
  float acc = __uint_as_float(0u);
  for (uint32_t base = 0; base < n; base += 2048) {
    const uint32_t cnt = n - base < 2048u ? n - base : 2048u;
    const uint32_t lo = base + 32 * lane;
    float v[32];
    if (lo + 32 <= n && (reinterpret_cast<uintptr_t>(s + lo) & 15u) == 0) {
      typedef float f4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f4 e = *reinterpret_cast<const f4*>(s + lo + 4 * i);
        v[4 * i + 0] = e[0];
        v[4 * i + 1] = e[1];
        v[4 * i + 2] = e[2];
        v[4 * i + 3] = e[3];
      }
    } else {
#pragma unroll
      for (int k = 0; k < 32; ++k) v[k] = lo + k < n ? s[lo + k] : 0.0f;
    }
    // every load has landed before the chain starts, so no wait sits in it
    __builtin_amdgcn_s_waitcnt(0);
    const uint32_t full = cnt / 32, rem = cnt % 32;
    for (uint32_t L = 0; L < full; ++L) {
      float a = acc;
      if (lane == L) {
#pragma unroll
        for (int k = 0; k < 32; ++k) a = a + v[k];
      }
      acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), (int)L));
    }
    if (rem) {
      float a = acc;
      if (lane == full) {
#pragma unroll
        for (int k = 0; k < 32; ++k)
          if ((uint32_t)k < rem) a = a + v[k];
      }
      acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), (int)full));
    }
  }
  return acc;
}

// The same fold with the running sum handed from lane to lane inside the
// vector unit (any n; s in LDS): each 2048-value chunk is held by the wave,
// lane L holding values 32L .. 32L+31 in registers.  Step L: every lane adds
// its own 32 values, in order, to the sum its left neighbour held after step
// L - 1 (lane 0 at step 0: the running sum), read through the first add's
// DPP source operand (wave_shr:1); only lane L's result is the fold's, the
// other lanes' are discarded.  No lane is masked off, so the chain carries
// no exec-mask updates, branches or scalar round trips: one dependent
// v_add_f32 per value (~4.5 cycles).  A chunk shorter than 2048 stops after
// its last lane holding values.  Every 16-byte chunk is loaded from an
// address inside [0, n) and replaced by +0 past the data, and the n % 4
// values past the last whole chunk are added last, in order, by the whole
// wave.  Slots past the data hold +0: the running sum starts at +0 and
// never becomes -0 (x + (-x) rounds to +0), so adding +0 leaves it
// unchanged and the bits equal serial_sum_wave's.  s not 16-byte aligned:
// serial_sum_wave.
CATENA_DEV float serial_sum_wave_long(const float* s, uint32_t n) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  if ((reinterpret_cast<uintptr_t>(s) & 15u) != 0) return serial_sum_wave(s, n);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t n4 = n & ~3u;  // values in whole 16-byte chunks
  float acc = __uint_as_float(0u);
  for (uint32_t base = 0; base < n4; base += 2048) {
    const uint32_t left = n4 - base;
    const uint32_t lo = base + 32 * lane;
    float v[32];
    if (left >= 2048u) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f4 q = *reinterpret_cast<const f4*>(s + lo + 4 * i);
#pragma unroll
        for (int j = 0; j < 4; ++j) v[4 * i + j] = q[j];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t e = lo + 4 * i;
        const bool in = e < n4;  // the whole chunk lies in [0, n4)
        const f4 q = *reinterpret_cast<const f4*>(s + (in ? e : 0u));
#pragma unroll
        for (int j = 0; j < 4; ++j) v[4 * i + j] = in ? q[j] : __uint_as_float(0u);
      }
    }
    // every load is issued and has landed before the chain starts, so no
    // wait sits inside it
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t nl = left >= 2048u ? 64u : (left + 31u) / 32u;
    float a = acc;
#pragma unroll
    for (int k = 0; k < 32; ++k) a = a + v[k];
    // lane L's 32 values after lane L-1's; eight lane blocks per loop
    // iteration, so that a taken branch sits in the chain once per 256
    // adds (2048 values: 11.4k -> 10.5k cycles)
    auto block = [&]() {
      // a DPP read of a VGPR needs two wait states after the VALU write of
      // it; across the loop's back edge only the branch separates them
      asm volatile("s_nop 1");
      a = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x138, 0xF, 0xF, true)) + v[0];
#pragma unroll
      for (int k = 1; k < 32; ++k) a = a + v[k];
    };
    uint32_t L = 1;
#pragma unroll 1
    for (; L + 8 <= nl; L += 8) {
#pragma unroll
      for (int r = 0; r < 8; ++r) block();
    }
#pragma unroll 1
    for (; L < nl; ++L) block();
    acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a), (int)(nl - 1)));
  }
  for (uint32_t t = n4; t < n; ++t) acc = acc + s[t];
  return acc;
}

// Cross-workgroup partial results.  The XCDs' L2 caches are not coherent
// with each other, so partials that another workgroup will read are stored
// and loaded as agent-scope atomics (relaxed): those bypass the non-coherent
// L2 state (write-through / coherent read) instead of writing back or
// invalidating whole caches with agent-scope fences.
CATENA_DEV void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
CATENA_DEV void store_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
CATENA_DEV float load_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
CATENA_DEV uint32_t load_coherent(const uint32_t* p) {
  return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Completion ticket shared by the workgroups of a group (e.g. the k-slices
// of one output tile).  Each workgroup calls it once, with all its threads,
// after writing its partials with store_coherent; it returns true in
// exactly one of them, the last to arrive, which then reads every partial of
// the group with load_coherent.  Ordering: each thread waits for its own
// stores to complete before the barrier, thread 0 takes the ticket with an
// agent-scope release (so the workgroup's partials are visible before the
// ticket moves), and the last workgroup's threads take an agent-scope acquire
// before they read, so no load of a partial is served from a stale cache
// line.  The last workgroup returns the counter to zero, so counters need
// clearing only once, when allocated.  Which workgroup reduces depends on
// timing; what it computes does not.
CATENA_DEV bool last_arrival(uint32_t* counter, uint32_t group_size, uint32_t* lds_flag) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t t =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t last = t == group_size - 1 ? 1u : 0u;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_flag = last;
  }
  __syncthreads();
  const bool last = *lds_flag != 0u;
  if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return last;
}

// Exact parallel form of the f32.max-env fold (catena-lang/stdlib/
// sum.hex:73-84: acc = (acc >= x) ? acc : x from acc = -inf, ascending).
// Without NaNs the fold returns the FIRST element that compares equal to the
// maximum (ties, including +0 == -0, keep the earlier one).  A NaN resets
// the fold: the result is then the last NaN itself if it is the final
// element, otherwise the first-max of the elements after the last NaN.
// Callers reduce (last_nan_index) first, then (value, index) pairs over the
// indices after it with first_max_combine, which is associative and
// commutative, so any reduction tree gives the sequential fold's bits.
struct FirstMax {
  float v;
  uint32_t i;  // 0xFFFFFFFF = empty (-inf sentinel)
};

CATENA_DEV FirstMax first_max_combine(FirstMax a, FirstMax b) {
  if (a.i == 0xFFFFFFFFu) return b;
  if (b.i == 0xFFFFFFFFu) return a;
  if (a.v > b.v) return a;
  if (b.v > a.v) return b;
  return (a.i < b.i) ? a : b;  // equal (incl. +0/-0): earlier index wins
}

// The same first maximum as one integer maximum: max_key orders (value,
// index) so that the largest key over non-NaN values is exactly the value
// first_max_combine keeps -- the value's bits made monotone (with -0 taken as
// +0, so equal values compare equal) above the complemented index (the
// earlier index wins), and the sign bit at the bottom so that the value's
// exact bits come back (key_score).  0 is below every key (no value).
// Index < 2^31.
CATENA_DEV uint32_t mono_bits(uint32_t bits) {
  const uint32_t canon = bits == 0x80000000u ? 0u : bits;
  return (canon & 0x80000000u) ? ~canon : (canon | 0x80000000u);
}
CATENA_DEV uint64_t make_key(uint32_t mono, uint32_t t, uint32_t bits) {
  return ((uint64_t)mono << 32) | ((0x7FFFFFFFu - t) << 1) | (bits >> 31);
}
CATENA_DEV uint64_t max_key(float v, uint32_t t) {
  const uint32_t bits = __float_as_uint(v);
  return make_key(mono_bits(bits), t, bits);
}

// Maximum over the wave of an unsigned value (0 is the identity): inclusive
// max scans within rows of 16 lanes (row_shr 1, 2, 4, 8), rows joined
// through row_bcast 15 and 31, lane 63's result returned uniformly.
CATENA_DEV uint32_t wave_umax(uint32_t x) {
#define CATENA_DPP_MAX(ctrl, rows) \
  x = max(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, (ctrl), (rows), 0xF, false))
  CATENA_DPP_MAX(0x111, 0xF);
  CATENA_DPP_MAX(0x112, 0xF);
  CATENA_DPP_MAX(0x114, 0xF);
  CATENA_DPP_MAX(0x118, 0xF);
  CATENA_DPP_MAX(0x142, 0xA);
  CATENA_DPP_MAX(0x143, 0xC);
#undef CATENA_DPP_MAX
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}
// Lane Q of each 16-lane row, broadcast to its row (DPP row_newbcast; the
// compiler folds it into the consuming VALU instruction's operand)
template <int Q>
CATENA_DEV float row_bcast16(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x150 + Q, 0xF, 0xF, false));
}
CATENA_DEV float key_score(uint64_t key) {
  const uint32_t mono = (uint32_t)(key >> 32);
  const uint32_t canon = (mono & 0x80000000u) ? (mono & 0x7FFFFFFFu) : ~mono;
  return __uint_as_float(canon == 0u ? ((uint32_t)key & 1u) << 31 : canon);
}
