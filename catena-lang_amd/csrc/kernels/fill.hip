// Seeded synthetic inputs for tests and benchmarks.
//
// Counter-based: element i of stream `stream` under `seed` is a pure
// function of (seed, stream, i), so any sub-range can be regenerated and the
// result does not depend on the launch shape.  u = splitmix64 finaliser of
// (seed * G + stream * S + i * G'); uniform = ((u >> 40) * 2^-24) * 2 - 1;
// normal = Box-Muller over two such uniforms, times `scale`, rounded to
// bf16 with round-to-nearest-even.
#include "common.h"

namespace {
CATENA_DEV uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
CATENA_DEV uint64_t draw(uint64_t seed, uint64_t stream, uint64_t i) {
  return mix64(seed * 0x9E3779B97F4A7C15ull + stream * 0xD1B54A32D192ED03ull +
               (i + 1) * 0xA0761D6478BD642Full);
}
CATENA_DEV float unit01(uint64_t u) {  // (0, 1]
  return (float)((u >> 40) + 1) * 5.9604644775390625e-8f;
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void catena_fill_uniform_f32(
    float* __restrict__ out, uint64_t n, uint64_t seed, uint64_t stream) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const uint64_t u = draw(seed, stream, i);
  out[i] = (float)(u >> 40) * 5.9604644775390625e-8f * 2.0f - 1.0f;
}

extern "C" __global__ __launch_bounds__(256) void catena_fill_normal_bf16(
    uint16_t* __restrict__ out, uint64_t n, uint64_t seed, uint64_t stream, float scale) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float u1 = unit01(draw(seed, stream, 2 * i));
  const float u2 = unit01(draw(seed, stream, 2 * i + 1));
  const float r = sqrtf(-2.0f * logf(u1));
  const float z = r * cosf(6.283185307179586f * u2);
  out[i] = (uint16_t)f32_to_bf16_bits(z * scale);
}

// Plain device-to-device copy in 16-byte units (n16 = bytes / 16): the
// reference kernel for calibrating HBM traffic counters, and a utility.
extern "C" __global__ __launch_bounds__(256) void catena_copy_16b(
    u32x4_t* __restrict__ dst, const u32x4_t* __restrict__ src, uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * 256;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride)
    dst[i] = __builtin_nontemporal_load(src + i);
}
