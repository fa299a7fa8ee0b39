// nn.softmax, math.exp-approx and the scalar stdlib maps as device kernels.
//
// nn.softmax (catena-lang/stdlib/nn.hex:93-122) over each of `rows` f32
// vectors of length n:
//   max   = f32.max-env fold from -inf          (catena-lang/stdlib/sum.hex:73-84)
//   denom = f32.add-env fold from +0 of exp~(x_i - max)   (nn.hex:59-72)
//   out_i = exp~(x_i - max) / denom                        (nn.hex:75-90)
// The reference runs both folds serially on the host (the entry is host-only
// because it contains a materialize).  Here one workgroup per row computes
// the max with the exact parallel form of the fold (FirstMax, common.h),
// writes exp~ values to the output, folds the denominator in ascending order
// as one lane-to-lane chain in wave 0 (serial_sum_wave), and divides in
// place -- bitwise the sequential result.
#include "common.h"

namespace {
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

extern "C" __global__ __launch_bounds__(256) void catena_softmax_rows_f32(
    const float* __restrict__ x, float* __restrict__ y, uint64_t n) {
  __shared__ int red_i[4];
  __shared__ float red_v[4];
  __shared__ uint32_t red_u[4];
  __shared__ float den_s;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* xr = x + (uint64_t)blockIdx.x * n;
  float* yr = y + (uint64_t)blockIdx.x * n;

  // index arithmetic of FirstMax is 32-bit; the host rejects n >= 2^32 - 1
  int lastnan = -1;
  for (uint64_t t = tid; t < n; t += 256)
    if (xr[t] != xr[t]) lastnan = (int)t;
  lastnan = wave_max_i32(lastnan);
  if (lane == 0) red_i[wave] = lastnan;
  __syncthreads();
  int J = red_i[0];
  for (int w = 1; w < 4; ++w) J = red_i[w] > J ? red_i[w] : J;

  FirstMax fm{__uint_as_float(0xFF800000u), 0xFFFFFFFFu};
  for (uint64_t t = tid; t < n; t += 256)
    if ((int64_t)t > J) fm = first_max_combine(fm, FirstMax{xr[t], (uint32_t)t});
  fm = wave_first_max(fm);
  if (lane == 0) {
    red_v[wave] = fm.v;
    red_u[wave] = fm.i;
  }
  __syncthreads();
  FirstMax all{red_v[0], red_u[0]};
  for (int w = 1; w < 4; ++w) all = first_max_combine(all, FirstMax{red_v[w], red_u[w]});
  float mx;
  if (n > 0 && J == (int64_t)n - 1)
    mx = xr[n - 1];
  else
    mx = (all.i == 0xFFFFFFFFu) ? __uint_as_float(0xFF800000u) : all.v;
  __syncthreads();  // x[n-1] is read above; y may alias x

  for (uint64_t t = tid; t < n; t += 256) {
    const float shifted = xr[t] - mx;
    yr[t] = exp_approx(shifted);
  }
  __syncthreads();
  if (tid < 64) {
    // den = (((0 + e_0) + e_1) + ...), ascending, as one lane-to-lane chain
    const float den = serial_sum_wave(yr, (uint32_t)n);
    if (tid == 0) den_s = den;
  }
  __syncthreads();
  const float den = den_s;
  for (uint64_t t = tid; t < n; t += 256) yr[t] = yr[t] / den;
}

// math.exp-approx applied elementwise (catena-lang/stdlib/math.hex:185-199).
extern "C" __global__ __launch_bounds__(256) void catena_exp_approx_f32(
    const float* __restrict__ x, float* __restrict__ y, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) y[i] = exp_approx(x[i]);
}

// The scalar stdlib programs applied elementwise, one device function each
// (common.h), selected by `op` (catena_map_op_t; uniform across the grid):
//   0 math.exp-approx       catena-lang/stdlib/math.hex:185-199
//   1 math.sqrt             catena-lang/stdlib/math.hex:235-272
//   2 nn.sigmoid            catena-lang/stdlib/nn.hex:1-12
//   3 nn.silu               catena-lang/stdlib/nn.hex:15-21
//   4 math.sin-approx       catena-lang/stdlib/math.hex:1-23
//   5 math.cos-approx       catena-lang/stdlib/math.hex:25-47
//   6 math.sin-approx-full  catena-lang/stdlib/math.hex:49-103
// The host rejects any other op before the launch.
extern "C" __global__ __launch_bounds__(256) void catena_map_f32(
    const float* __restrict__ x, float* __restrict__ y, uint64_t n, uint32_t op) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  float r;
  switch (op) {
    case 0: r = exp_approx(v); break;
    case 1: r = sqrt_newton(v); break;
    case 2: r = sigmoid_approx(v); break;
    case 3: r = silu_approx(v); break;
    case 4: r = sin_taylor(v); break;
    case 5: r = cos_taylor(v); break;
    default: r = sin_full(v); break;
  }
  y[i] = r;
}
