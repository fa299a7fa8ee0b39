// The reference's materializec producers and reducec folds over buffers
// (catena-lang/stdlib/tensor.hex:1-168, catena-lang/stdlib/sum.hex:7-101),
// as device kernels with the reference's element order:
//   tensor.broadcast-f32   out[i] = value
//   tensor.arange-f32      out[i] = u64.to-f32(i)            (RNE)
//   tensor.slice-f32 / tensor.concat-f32: element copies (catena_copy_f32)
//   sum-f32 / mean-f32     acc = fold_{i asc} from +0 of acc + x_i
//                          (mean: then acc / u64.to-f32(n))
//   max-f32                f32.max-env fold from -inf (acc >= x ? acc : x)
//   sum-u64 / dot-u64      wrapping u64 sums (order-independent), the
//                          reference's test programs tests/cases/reducec/basic.hex
// The f32 sum stays one serial chain (serial_sum_wave); the max uses the
// exact parallel form of its fold (FirstMax in common.h).
#include "common.h"

namespace {
CATENA_DEV int wave_max_i32(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const int o = __shfl_xor(v, off, 64);
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

CATENA_DEV uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), off, 64) << 32) |
                       (uint32_t)__shfl_xor((int)(uint32_t)v, off, 64);
    v = v + o;
  }
  return v;
}
}  // namespace

// grid-stride producers, block 256
extern "C" __global__ __launch_bounds__(256) void catena_broadcast_f32(float* __restrict__ out,
                                                                       uint64_t n, float value) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) out[i] = value;
}

extern "C" __global__ __launch_bounds__(256) void catena_arange_f32(float* __restrict__ out,
                                                                    uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    out[i] = (float)i;  // u64.to-f32: round to nearest even
}

// dst[i] = src[i], i < n (4-byte elements, any 4-byte alignment)
extern "C" __global__ __launch_bounds__(256) void catena_copy_f32(float* __restrict__ dst,
                                                                  const float* __restrict__ src,
                                                                  uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

// sum-f32 (mean = 0: the sum; mean = 1: sum / (f32)n) of each row; one
// wave per row.
extern "C" __global__ __launch_bounds__(64) void catena_sum_rows_f32(
    const float* __restrict__ x, float* __restrict__ out, uint64_t n, uint32_t mean) {
  const float* xr = x + (uint64_t)blockIdx.x * n;
  const float sum = serial_sum_wave(xr, (uint32_t)n);
  if (threadIdx.x == 0) {
    if (mean) {
      const float len_f = (float)n;
      out[blockIdx.x] = sum / len_f;
    } else {
      out[blockIdx.x] = sum;
    }
  }
}

// max-f32 of each row: the f32.max-env fold from -inf.  A NaN replaces the
// accumulator and the next element replaces the NaN, so the result is the
// last NaN when it is the final element, else the first maximum of the
// elements after the last NaN (or -inf when there are none).
extern "C" __global__ __launch_bounds__(256) void catena_max_rows_f32(
    const float* __restrict__ x, float* __restrict__ out, uint64_t n) {
  __shared__ int red_i[4];
  __shared__ float red_v[4];
  __shared__ uint32_t red_u[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* xr = x + (uint64_t)blockIdx.x * n;
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
  if (tid != 0) return;
  FirstMax all{red_v[0], red_u[0]};
  for (int w = 1; w < 4; ++w) all = first_max_combine(all, FirstMax{red_v[w], red_u[w]});
  float mx;
  if (n > 0 && J == (int64_t)n - 1)
    mx = xr[n - 1];
  else
    mx = (all.i == 0xFFFFFFFFu) ? __uint_as_float(0xFF800000u) : all.v;
  out[blockIdx.x] = mx;
}

// sum-u64 (b == NULL) or dot-u64 of a row: wrapping u64 arithmetic, so any
// summation order gives the reference's value.
extern "C" __global__ __launch_bounds__(256) void catena_sum_rows_u64(
    const uint64_t* __restrict__ a, const uint64_t* __restrict__ b, uint64_t* __restrict__ out,
    uint64_t n) {
  __shared__ uint64_t red[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint64_t* ar = a + (uint64_t)blockIdx.x * n;
  const uint64_t* br = b ? b + (uint64_t)blockIdx.x * n : nullptr;
  uint64_t acc = 0;
  for (uint64_t t = tid; t < n; t += 256) acc += br ? ar[t] * br[t] : ar[t];
  acc = wave_sum_u64(acc);
  if (lane == 0) red[wave] = acc;
  __syncthreads();
  if (tid == 0) out[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}
