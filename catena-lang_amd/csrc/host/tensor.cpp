// Kernel and program ABI of the reference's buffer producers and folds
// (catena-lang/stdlib/tensor.hex:1-168, catena-lang/stdlib/sum.hex:7-101,
// catena-lang/tests/cases/reducec/basic.hex).
#include <cstdint>

#include "internal.h"

using namespace catena;

namespace {
uint64_t ceil_div(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// grid of at most 65536 workgroups of 256 for the grid-stride kernels
unsigned stride_grid(uint64_t n) {
  const uint64_t g = ceil_div(n, 256);
  return (unsigned)(g < 65536 ? g : 65536);
}

int rows_ok(uint64_t rows, uint64_t n, uint64_t max_n, const char* what) {
  if (rows > 0x7FFFFFFFull) return fail(CATENA_ERR_UNSUPPORTED, "%s: too many rows", what);
  if (n > max_n) return fail(CATENA_ERR_UNSUPPORTED, "%s: rows of %llu elements exceed %llu", what,
                             (unsigned long long)n, (unsigned long long)max_n);
  return CATENA_OK;
}

void check(int status, const char* what) {
  if (status != CATENA_OK) trap_gpu(what);
}

catena_mem_t alloc_out(uint64_t bytes) {
  catena_mem_t m{nullptr, 0};
  check(catena_mem_alloc(bytes, &m), "output allocation");
  return m;
}

uint64_t add_or_trap(uint64_t a, uint64_t b) {
  uint64_t r;
  if (__builtin_add_overflow(a, b, &r)) trap_assert("size overflow");
  return r;
}
}  // namespace

extern "C" {

int catena_mi355x_broadcast_f32(float* out, uint64_t n, float value) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  void* args[] = {&out, &n, &value};
  return launch(KernelId::BroadcastF32, dim3(stride_grid(n)), dim3(256), 0, args);
}

int catena_mi355x_arange_f32(float* out, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!out) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  void* args[] = {&out, &n};
  return launch(KernelId::ArangeF32, dim3(stride_grid(n)), dim3(256), 0, args);
}

int catena_mi355x_copy_f32(float* dst, const float* src, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (n == 0) return CATENA_OK;
  if (!dst || !src) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  void* args[] = {&dst, &src, &n};
  return launch(KernelId::CopyF32, dim3(stride_grid(n)), dim3(256), 0, args);
}

// Longest f32 sum row: the one-wave serial fold walks a row in 32-bit
// 2048-value chunks (chunk base and lane offsets must not wrap).
constexpr uint64_t kSumMaxN = 0xFFFFF800ull;

static int sum_launch(const float* x, float* out, uint64_t rows, uint64_t n, uint32_t mean) {
  if (rows == 0) return ensure_init();
  if (!out || (n > 0 && !x)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  int st = rows_ok(rows, n, kSumMaxN, "sum-f32");
  if (st) return st;
  st = ensure_init();
  if (st) return st;
  void* args[] = {&x, &out, &n, &mean};
  return launch(KernelId::SumRowsF32, dim3((unsigned)rows), dim3(64), 0, args);
}

int catena_mi355x_sum_f32(const float* x, float* out, uint64_t rows, uint64_t n) {
  return sum_launch(x, out, rows, n, 0);
}

int catena_mi355x_mean_f32(const float* x, float* out, uint64_t rows, uint64_t n) {
  return sum_launch(x, out, rows, n, 1);
}

int catena_mi355x_max_f32(const float* x, float* out, uint64_t rows, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0) return CATENA_OK;
  if (!out || (n > 0 && !x)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  st = rows_ok(rows, n, 0x7FFFFFFEull, "max-f32");
  if (st) return st;
  void* args[] = {&x, &out, &n};
  return launch(KernelId::MaxRowsF32, dim3((unsigned)rows), dim3(256), 0, args);
}

int catena_mi355x_sum_u64(const uint64_t* x, uint64_t* out, uint64_t rows, uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0) return CATENA_OK;
  if (!out || (n > 0 && !x)) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  st = rows_ok(rows, n, ~0ull, "sum-u64");
  if (st) return st;
  const uint64_t* b = nullptr;
  void* args[] = {&x, &b, &out, &n};
  return launch(KernelId::SumRowsU64, dim3((unsigned)rows), dim3(256), 0, args);
}

int catena_mi355x_dot_u64(const uint64_t* a, const uint64_t* b, uint64_t* out, uint64_t rows,
                          uint64_t n) {
  int st = ensure_init();
  if (st) return st;
  if (rows == 0) return CATENA_OK;
  if (!out || (n > 0 && (!a || !b))) return fail(CATENA_ERR_INVALID_ARGUMENT, "null operand");
  st = rows_ok(rows, n, ~0ull, "dot-u64");
  if (st) return st;
  void* args[] = {&a, &b, &out, &n};
  return launch(KernelId::SumRowsU64, dim3((unsigned)rows), dim3(256), 0, args);
}

// ---------------------------------------------------------------- programs

void program_tensor_broadcast_f32(float value, uint64_t len, catena_mem_t* out) {
  if (len > (~0ull) / 4) trap_assert("size overflow");
  catena_mem_t m = alloc_out(len * 4);
  check(catena_mi355x_broadcast_f32(static_cast<float*>(m.data), len, value), "tensor.broadcast-f32");
  check(catena_mi355x_synchronize(), "synchronize");
  *out = m;
}

void program_tensor_arange_f32(uint64_t len, catena_mem_t* out) {
  if (len > (~0ull) / 4) trap_assert("size overflow");
  catena_mem_t m = alloc_out(len * 4);
  check(catena_mi355x_arange_f32(static_cast<float*>(m.data), len), "tensor.arange-f32");
  check(catena_mi355x_synchronize(), "synchronize");
  *out = m;
}

void program_tensor_slice_f32(catena_mem_t input, uint64_t start, uint64_t len, catena_mem_t* out) {
  // tensor.slice-at asserts start + i < len(input) for every output index
  // (catena-lang/stdlib/tensor.hex:49-66); checked once, before the copy.
  const uint64_t in_len = input.len / 4;  // mem.cast.f32
  if (len > 0 && (add_or_trap(start, len) > in_len)) trap_assert("start + i < len(input)");
  catena_mem_t m = alloc_out(len * 4);
  if (len > 0) {
    check(catena_mi355x_copy_f32(static_cast<float*>(m.data),
                                 static_cast<const float*>(input.data) + start, len),
          "tensor.slice-f32");
    check(catena_mi355x_synchronize(), "synchronize");
  }
  *out = m;
}

void program_tensor_concat_f32(catena_mem_t a, catena_mem_t b, catena_mem_t* out) {
  const uint64_t la = a.len / 4, lb = b.len / 4;
  const uint64_t total = add_or_trap(la, lb);
  catena_mem_t m = alloc_out(total * 4);
  float* dst = static_cast<float*>(m.data);
  if (la) check(catena_mi355x_copy_f32(dst, static_cast<const float*>(a.data), la), "tensor.concat-f32");
  if (lb)
    check(catena_mi355x_copy_f32(dst + la, static_cast<const float*>(b.data), lb), "tensor.concat-f32");
  check(catena_mi355x_synchronize(), "synchronize");
  *out = m;
}

static float fold_program(catena_mem_t x, int which) {
  const uint64_t n = x.len / 4;
  catena_mem_t r = alloc_out(4);
  const float* p = static_cast<const float*>(x.data);
  float* o = static_cast<float*>(r.data);
  int st = which == 0 ? catena_mi355x_sum_f32(p, o, 1, n)
         : which == 1 ? catena_mi355x_mean_f32(p, o, 1, n)
                      : catena_mi355x_max_f32(p, o, 1, n);
  check(st, which == 0 ? "sum-f32" : which == 1 ? "mean-f32" : "max-f32");
  float v = 0.0f;
  check(catena_mem_read(r, 0, &v, 4), "download");
  catena_mem_free(&r);
  return v;
}

void program_sum_f32(catena_mem_t x, float* out) { *out = fold_program(x, 0); }
void program_mean_f32(catena_mem_t x, float* out) { *out = fold_program(x, 1); }
void program_max_f32(catena_mem_t x, float* out) { *out = fold_program(x, 2); }

void program_sum_u64(catena_mem_t x, uint64_t* out) {
  catena_mem_t r = alloc_out(8);
  check(catena_mi355x_sum_u64(static_cast<const uint64_t*>(x.data), static_cast<uint64_t*>(r.data),
                              1, x.len / 8),
        "sum-u64");
  check(catena_mem_read(r, 0, out, 8), "download");
  catena_mem_free(&r);
}

void program_dot_u64(catena_mem_t a, catena_mem_t b, uint64_t* out) {
  // mem.cast.u64.same-length (tests/cases/reducec/basic.hex): equal lengths
  if (a.len / 8 != b.len / 8) trap_assert("len(lhs) == len(rhs)");
  catena_mem_t r = alloc_out(8);
  check(catena_mi355x_dot_u64(static_cast<const uint64_t*>(a.data),
                              static_cast<const uint64_t*>(b.data), static_cast<uint64_t*>(r.data),
                              1, a.len / 8),
        "dot-u64");
  check(catena_mem_read(r, 0, out, 8), "download");
  catena_mem_free(&r);
}

}  // extern "C"
