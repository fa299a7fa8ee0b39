// Program ABI: the `program_<name>` entry points of catena's generated
// module, re-implemented on the native kernels.
//
// Contract (catena-lang/src/codegen/gpu.rs:235-285,
// catena-lang/src/runtime/executor.rs:88-106): inputs by value, outputs
// through pointers, void return, synchronous.  Inputs are borrowed; outputs
// are freshly allocated (here from the pool) and owned by the caller, who
// releases them with catena_mem_free (reference: Mem::drop,
// catena-lang/src/runtime/mem.rs:119-125).  Failed assertions and GPU errors
// print and trap (catena-lang/src/codegen/prelude.rs:38-55).
#include <cstdio>
#include <cstdlib>

#include "internal.h"

namespace catena {

void trap_assert(const char* what) {
  fprintf(stderr, "catena assertion failed: %s\n", what);
  fflush(stderr);
  __builtin_trap();
}

void trap_gpu(const char* what) {
  fprintf(stderr, "catena GPU error: %s: %s\n", what, last_error());
  fflush(stderr);
  __builtin_trap();
}

}  // namespace catena

using namespace catena;

namespace {
void check(int status, const char* what) {
  if (status != CATENA_OK) trap_gpu(what);
}

void sync_or_trap() { check(catena_mi355x_synchronize(), "synchronize"); }

// Multiplications of caller-supplied sizes are checked so a bad size traps
// instead of wrapping.
uint64_t mul_or_trap(uint64_t a, uint64_t b) {
  uint64_t r;
  if (__builtin_mul_overflow(a, b, &r)) trap_assert("size overflow");
  return r;
}

// Output of materializec: a fresh owned buffer of `bytes` (data == NULL
// when empty, catena-lang/src/codegen/ops/materializec.rs:113-122).
catena_mem_t alloc_out(uint64_t bytes) {
  catena_mem_t m{nullptr, 0};
  check(catena_mem_alloc(bytes, &m), "output allocation");
  return m;
}

// f32.matrix.identity (catena-lang/stdlib/matrix.hex:129-159):
// I(i, j) = (i != j) ? +0.0f : 1.0f, materialised on the device.
catena_mem_t identity_f32(uint64_t n) {
  const uint64_t cells = mul_or_trap(n, n);
  catena_mem_t m = alloc_out(mul_or_trap(cells, 4));
  if (cells == 0) return m;
  float* host = static_cast<float*>(calloc(cells, sizeof(float)));
  if (!host) trap_assert("host allocation for identity");
  for (uint64_t i = 0; i < n; ++i) host[i * n + i] = 1.0f;
  check(catena_mem_write(m, 0, host, cells * 4), "identity upload");
  free(host);
  return m;
}

// A scalar (f32) -> (f32) program on the device: the value goes up, one
// thread applies the op, the result comes back.
void scalar_map(uint32_t op, float x, float* out, const char* what) {
  catena_mem_t buf = alloc_out(8);
  check(catena_mem_write(buf, 0, &x, 4), "upload");
  float* p = static_cast<float*>(buf.data);
  check(catena_mi355x_map_f32(op, p, p + 1, 1), what);
  check(catena_mem_read(buf, 4, out, 4), "download");
  catena_mem_free(&buf);
}

void matmul_f32_mem(const void* a, const void* b, uint64_t n, uint64_t m, uint64_t k,
                    catena_mem_t* out) {
  catena_mem_t c = alloc_out(mul_or_trap(mul_or_trap(n, m), 4));
  check(catena_mi355x_gemm_f32_exact(static_cast<const float*>(a), static_cast<const float*>(b),
                                     static_cast<float*>(c.data), n, m, k),
        "f32 matmul");
  sync_or_trap();
  *out = c;
}
}  // namespace

extern "C" {

void program_matmul_2x2_via_mem(catena_mem_t a, catena_mem_t b, uint64_t n, uint64_t m,
                                uint64_t k, uint64_t nk, uint64_t km, uint64_t nm,
                                catena_mem_t* out) {
  // mem.cast.f32 (len = bytes / 4, catena-lang/src/codegen/gpu.rs:768-782),
  // then the two u64.eq + assert-then checks of tests/cases/matrix/matmul.hex:16-29.
  if (nk != a.len / 4) trap_assert("nk == len(a)");
  if (km != b.len / 4) trap_assert("km == len(b)");
  // Value-level shape checks the reference leaves to its dependent types.
  if (mul_or_trap(n, k) != nk || mul_or_trap(k, m) != km || mul_or_trap(n, m) != nm)
    trap_assert("n*k == nk, k*m == km, n*m == nm");
  matmul_f32_mem(a.data, b.data, n, m, k, out);
}

void program_matmul_right_identity_2x2_via_mem(catena_mem_t a, uint64_t n, uint64_t nn,
                                               catena_mem_t* out) {
  if (nn != a.len / 4) trap_assert("nn == len(a)");
  if (mul_or_trap(n, n) != nn) trap_assert("n*n == nn");
  catena_mem_t id = identity_f32(n);
  matmul_f32_mem(a.data, id.data, n, n, n, out);
  catena_mem_free(&id);
}

void program_matmul_left_identity_2x2_via_mem(catena_mem_t a, uint64_t n, uint64_t nn,
                                              catena_mem_t* out) {
  if (nn != a.len / 4) trap_assert("nn == len(a)");
  if (mul_or_trap(n, n) != nn) trap_assert("n*n == nn");
  catena_mem_t id = identity_f32(n);
  matmul_f32_mem(id.data, a.data, n, n, n, out);
  catena_mem_free(&id);
}

void program_nn_softmax(catena_mem_t x, catena_mem_t* out) {
  const uint64_t n = x.len / 4;  // mem.cast.f32
  catena_mem_t y = alloc_out(n * 4);
  check(catena_mi355x_softmax_f32(static_cast<const float*>(x.data), static_cast<float*>(y.data), 1,
                                  n),
        "nn.softmax");
  sync_or_trap();
  *out = y;
}

void program_math_exp_approx(float x, float* out) {
  catena_mem_t buf = alloc_out(8);
  check(catena_mem_write(buf, 0, &x, 4), "upload");
  float* p = static_cast<float*>(buf.data);
  check(catena_mi355x_exp_approx_f32(p, p + 1, 1), "math.exp-approx");
  check(catena_mem_read(buf, 4, out, 4), "download");
  catena_mem_free(&buf);
}

void program_math_sqrt(float x, float* out) { scalar_map(CATENA_MAP_SQRT, x, out, "math.sqrt"); }
void program_nn_sigmoid(float x, float* out) { scalar_map(CATENA_MAP_SIGMOID, x, out, "nn.sigmoid"); }
void program_nn_silu(float x, float* out) { scalar_map(CATENA_MAP_SILU, x, out, "nn.silu"); }
void program_math_sin_approx(float x, float* out) {
  scalar_map(CATENA_MAP_SIN_APPROX, x, out, "math.sin-approx");
}
void program_math_cos_approx(float x, float* out) {
  scalar_map(CATENA_MAP_COS_APPROX, x, out, "math.cos-approx");
}
void program_math_sin_approx_full(float x, float* out) {
  scalar_map(CATENA_MAP_SIN_APPROX_FULL, x, out, "math.sin-approx-full");
}

void program_bf16_matmul_via_mem(catena_mem_t a, catena_mem_t b, uint64_t n, uint64_t m,
                                 uint64_t k, uint64_t nk, uint64_t km, uint64_t nm,
                                 catena_mem_t* out) {
  if (nk != a.len / 2) trap_assert("nk == len(a)");
  if (km != b.len / 2) trap_assert("km == len(b)");
  if (mul_or_trap(n, k) != nk || mul_or_trap(k, m) != km || mul_or_trap(n, m) != nm)
    trap_assert("n*k == nk, k*m == km, n*m == nm");
  catena_mem_t c = alloc_out(mul_or_trap(nm, 2));
  check(catena_mi355x_gemm_bf16(static_cast<const uint16_t*>(a.data),
                                static_cast<const uint16_t*>(b.data), c.data, n, m, k, 0),
        "bf16 matmul");
  sync_or_trap();
  *out = c;
}

void program_attn_decode_via_mem(catena_mem_t q, catena_mem_t k, catena_mem_t v,
                                 catena_mem_t lens, uint64_t batch, uint64_t heads,
                                 uint64_t max_len, uint64_t head_dim, float scale,
                                 catena_mem_t* out) {
  if (batch > 0xFFFFFFFFull || heads > 0xFFFFFFFFull || max_len > 0xFFFFFFFFull ||
      head_dim > 0xFFFFFFFFull)
    trap_assert("sizes fit u32");
  const uint64_t bhd = mul_or_trap(mul_or_trap(batch, heads), head_dim);
  if (q.len != mul_or_trap(bhd, 2)) trap_assert("len(q) == batch*heads*head_dim*2");
  const uint64_t kv = mul_or_trap(mul_or_trap(bhd, max_len), 2);
  if (k.len != kv || v.len != kv) trap_assert("len(k) == len(v) == batch*heads*max_len*head_dim*2");
  if (lens.len != mul_or_trap(batch, 4)) trap_assert("len(lens) == batch*4");
  if (batch > 0) {
    uint32_t* host = static_cast<uint32_t*>(malloc(lens.len));
    if (!host) trap_assert("host allocation for lens");
    check(catena_mem_read(lens, 0, host, lens.len), "lens download");
    for (uint64_t i = 0; i < batch; ++i)
      if (host[i] > max_len) trap_assert("lens[i] <= max_len");
    free(host);
  }
  catena_mem_t o = alloc_out(mul_or_trap(bhd, 4));
  check(catena_mi355x_attn_decode_bf16(
            static_cast<const uint16_t*>(q.data), static_cast<const uint16_t*>(k.data),
            static_cast<const uint16_t*>(v.data), static_cast<const uint32_t*>(lens.data),
            static_cast<float*>(o.data), (uint32_t)batch, (uint32_t)heads, (uint32_t)max_len,
            (uint32_t)head_dim, scale),
        "attention decode");
  sync_or_trap();
  *out = o;
}

}  // extern "C"
